"""Python bindings of librkhip (include/rk.h) over ctypes.

This is host plumbing for tests and benchmarks: every computation runs in
librkhip.so's HIP kernels. Loading fails loudly when the library is not
built; there is no CPU fallback.
"""
import ctypes
import os

import numpy as np

# The error type is the broker worker module's (librkworker.so, host only),
# so a status from either library is one class to catch.
from rkworker import RKError

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "librkhip.so")
HEADER = os.path.join(os.path.dirname(PKG_DIR), "include", "rk.h")

RK_OK, RK_ERR_ARGS, RK_ERR_OOM, RK_ERR_HIP, RK_ERR_UNSUPPORTED, RK_ERR_NO_DEVICE = 0, -1, -2, -3, -4, -5
F32, BF16, Q8, Q4, FP8, FP4 = 0, 1, 2, 3, 4, 5

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
F = ctypes.c_float

_lib = None


class DeviceInfo(ctypes.Structure):
    _fields_ = [("index", I32), ("name", ctypes.c_char * 64), ("arch", ctypes.c_char * 32), ("memory", I64),
                ("compute_units", I32), ("exact", I32), ("integrated", I32)]


# name -> (restype, argtypes); the exported C-ABI, kept in step with rk.h.
SIGNATURES = {
    "rk_device_count": (ctypes.c_int, [P]),
    "rk_device_info_get": (ctypes.c_int, [I32, P]),
    "rk_device_open": (ctypes.c_int, [I32, P]),
    "rk_device_close": (ctypes.c_int, [P]),
    "rk_used_bytes": (I64, [P]),
    "rk_last_error": (ctypes.c_char_p, [P]),
    "rk_matrix_upload": (ctypes.c_int, [P, I32, I64, I64, P, P, P]),
    "rk_matrix_free": (ctypes.c_int, [P]),
    "rk_matrix_upload_mx": (ctypes.c_int, [P, I32, I64, I64, P, P, P]),
    "rk_matrix_set_raw": (ctypes.c_int, [P, I32]),
    "rk_matrix_upload_mx_chunks": (ctypes.c_int, [P, I32, I64, I64, I32, P, P, I32, P, P, I32, P]),
    "rk_batch_quantize_fp8": (ctypes.c_int, [P, I64, I64]),
    "rk_batch_expert_matvecs": (ctypes.c_int, [P, P, I64, I64, I32, I64, I64, I32, I64, I64]),
    "rk_batch_matvecs_batch": (ctypes.c_int, [P, P, I64, I64, I64, I64, I32]),
    "rk_batch_act_quant_inplace": (ctypes.c_int, [P, I64, I64]),
    "rk_batch_fp4_quant_inplace": (ctypes.c_int, [P, I64, I64, I32]),
    "rk_matrix_bytes": (I64, [P]),
    "rk_matvecs": (ctypes.c_int, [P, I32, P, P, P, I64]),
    "rk_matvecs_device": (ctypes.c_int, [P, I32, P, P, P, I64, P]),
    "rk_matmul_t": (ctypes.c_int, [P, I32, P, P, P, I64, I32]),
    "rk_matmul_t_device": (ctypes.c_int, [P, I32, P, P, P, I64, I32, P]),
    "rk_matmul_t_device_noalloc": (ctypes.c_int, [P, I32, P, P, P, I64, I32, P]),
    "rk_arena_new": (ctypes.c_int, [P, I64, I64, P]),
    "rk_arena_set_quant_scratch": (ctypes.c_int, [P, I64, I64]),
    "rk_arena_bytes": (I64, [P]),
    "rk_arena_free": (ctypes.c_int, [P]),
    "rk_arena_device_ptr": (ctypes.c_int, [P, I64, P]),
    "rk_vectors_upload": (ctypes.c_int, [P, P, I64, P]),
    "rk_vectors_free": (ctypes.c_int, [P]),
    "rk_batch_begin": (ctypes.c_int, [P, P]),
    "rk_batch_write": (ctypes.c_int, [P, I64, P, I64]),
    "rk_batch_read": (ctypes.c_int, [P, I64, P, I64]),
    "rk_batch_matvecs": (ctypes.c_int, [P, I32, P, P, I64]),
    "rk_batch_quantize": (ctypes.c_int, [P, I64, I64]),
    "rk_batch_rmsnorm": (ctypes.c_int, [P, P, I64, I64, I64, I32, I32, I64, F, F]),
    "rk_batch_addvec": (ctypes.c_int, [P, P, I64, I64, I64]),
    "rk_batch_rope": (ctypes.c_int, [P, I64, I64, I32, I32, I32, I64, I64]),
    "rk_batch_copy": (ctypes.c_int, [P, I64, I64, I64]),
    "rk_batch_attention": (ctypes.c_int, [P, I64, I64, I64, I64, I64, I64, I32, I32, I32, I32, I32, F]),
    "rk_batch_residual": (ctypes.c_int, [P, I64, I64, I64, I32]),
    "rk_batch_silumul": (ctypes.c_int, [P, I64, I64, I64]),
    "rk_batch_submit": (ctypes.c_int, [P]),
    "rk_graph_begin": (ctypes.c_int, [P]),
    "rk_graph_end": (ctypes.c_int, [P, P]),
    "rk_graph_launch": (ctypes.c_int, [P, I32]),
    "rk_graph_launch_timed": (ctypes.c_int, [P, I32, P]),
    "rk_graph_free": (ctypes.c_int, [P]),
    "rk_profile_start": (ctypes.c_int, [P]),
    "rk_profile_stop": (ctypes.c_int, [P, P, I32, P]),
    "rk_device_launch_floor": (ctypes.c_int, [P, I64, I32, I32, P, P]),
    "rk_tensor_serve": (ctypes.c_int, [P, I32, I64]),
    "rk_stage_new": (ctypes.c_int, [P, P, P, I32, P, P, P]),
    "rk_stage_forward": (ctypes.c_int, [P, P, I32, I32]),
    "rk_stage_bytes": (I64, [P]),
    "rk_stage_free": (ctypes.c_int, [P]),
    "rk_stage_set_head": (ctypes.c_int, [P, P, P, P]),
    "rk_stage_generate_start": (ctypes.c_int, [P, P, I32]),
    "rk_stage_generate_run": (ctypes.c_int, [P, I32, P]),
    "rk_stage_generate_tokens": (ctypes.c_int, [P, I32, I32, P]),
    "rk_stage_generate": (ctypes.c_int, [P, P, I32, I32, P]),
    "rk_stage_seqs_start": (ctypes.c_int, [P, P, P]),
    "rk_stage_seqs_run": (ctypes.c_int, [P, I32, P]),
    "rk_stage_seqs_tokens": (ctypes.c_int, [P, I32, I32, I32, P]),
    "rk_stage_sampler": (ctypes.c_int, [P, I32, ctypes.c_float, ctypes.c_uint64]),
    "rk_sample_logits": (ctypes.c_int, [P, P, I64, I32, P, P, P]),
    "rk_stage_moe_stats": (ctypes.c_int, [P, P, P]),
    "rk_num_eval": (ctypes.c_int, [P, I32, P, P, I64]),
    "rk_moe_new": (ctypes.c_int, [P, P, I32, P, P, P, I32, P]),
    "rk_moe_ffn": (ctypes.c_int, [P, P, I32, P, P, P]),
    "rk_moe_ffn_device": (ctypes.c_int, [P, P, I32, P, P]),
    "rk_moe_bytes": (I64, [P]),
    "rk_moe_free": (ctypes.c_int, [P]),
    "rk_tensor_matmul": (ctypes.c_int, [P, I32, I32, I64, I64, I64, P, P, P]),
    "rk_tensor_matmul_device": (ctypes.c_int, [P, I32, I32, I64, I64, I64, P, P, P, P]),
    "rk_tensor_quantize": (ctypes.c_int, [P, P, P, I64, ctypes.c_float]),
    "rk_tensor_scale": (ctypes.c_int, [P, I32, P, P, I64, ctypes.c_float]),
}

TENSOR_F32, TENSOR_I8, TENSOR_I32 = 0, 1, 2

FN_RECIP32, FN_RSQRT32, FN_EXP32, FN_SILU = 0, 1, 2, 3


class StageConfig(ctypes.Structure):
    """rk_stage_config (include/rk.h)."""
    _fields_ = [(n, I32) for n in ("dim", "hidden", "heads", "kv_heads", "head_dim", "ctx", "qkv_bias", "qk_norm")] + \
               [(n, F) for n in ("norm_eps", "recip_dim", "recip_head", "inv_sqrt")] + [("seqs", I32)]


class StageLayer(ctypes.Structure):
    """rk_stage_layer (include/rk.h)."""
    _fields_ = [(n, P) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att", "rms_ffn", "bq", "bk", "bv",
                                 "q_norm", "k_norm", "moe")]


def inv_sqrt_head(hs):
    """The attention scores' scale as the Go host computes it
    (internal/llm/model.go:529, gpustage.go:125):
    float32(1/math.Sqrt(float64(hs))), a float64 square root and division
    (each correctly rounded) rounded once more to float32."""
    return np.float32(1.0 / np.sqrt(np.float64(hs)))


def lib():
    """The loaded librkhip.so; raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() (hipcc, gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(P)


def device_count():
    n = I32()
    lib().rk_device_count(ctypes.byref(n))
    return n.value


def devices():
    """internal/gpu/device.go:125-183 Devices: every device's info."""
    return [device_info(i) for i in range(device_count())]


def best(infos):
    """internal/gpu/device.go:185-201 Best: among devices computing exactly,
    the discrete one with the most memory, else an integrated one; None if
    none is exact."""
    pick = None
    for d in infos:
        if not d.exact:
            continue
        rank = 2 if d.integrated else 3
        if pick is None or rank > pick[0] or (rank == pick[0] and d.memory > pick[1].memory):
            pick = (rank, d)
    return pick[1] if pick else None


def tensor_call(fd, a, b, transposed=False):
    """The worker side of the tensor broker, as rkworker.tensor_call (which
    a worker process imports alone: librkworker.so, no GPU runtime)."""
    import rkworker

    return rkworker.tensor_call(fd, a, b, transposed)


def device_bytes_budget(info):
    """internal/llm/service.go:210-212: the default budget of a node's GPU
    layers, 85 % of the device's memory (memory / 100 * 85 in integers)."""
    return int(info.memory) // 100 * 85


def device_info(index=0):
    info = DeviceInfo()
    rc = lib().rk_device_info_get(index, ctypes.byref(info))
    if rc != RK_OK:
        raise RKError(rc, lib().rk_last_error(None).decode())
    return info


class ProfileEntry(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_char * 48), ("calls", I64), ("ms", ctypes.c_double)]


class Matrix:
    def __init__(self, dev, handle, kind, rows, cols):
        self.dev, self.h, self.kind, self.rows, self.cols = dev, handle, kind, rows, cols

    @property
    def bytes(self):
        return lib().rk_matrix_bytes(self.h)

    def set_raw(self, raw):
        """E4M3 / E2M1 products left in float32 (internal/gpu Matrix.unrounded)."""
        self.dev._check(lib().rk_matrix_set_raw(self.h, int(bool(raw))))

    def free(self):
        if self.h:
            self.dev._check(lib().rk_matrix_free(self.h))
            self.h = None


class Vectors:
    def __init__(self, dev, handle, n):
        self.dev, self.h, self.n = dev, handle, n

    def free(self):
        if self.h:
            self.dev._check(lib().rk_vectors_free(self.h))
            self.h = None


class Arena:
    """Device words for a computation (internal/gpu Arena)."""

    def __init__(self, dev, words, staging_words):
        self.dev = dev
        h = P()
        dev._check(lib().rk_arena_new(dev.h, words, staging_words, ctypes.byref(h)))
        self.h, self.words = h, words

    def set_quant_scratch(self, qx_off, xs_off):
        self.dev._check(lib().rk_arena_set_quant_scratch(self.h, qx_off, xs_off))

    @property
    def bytes(self):
        return lib().rk_arena_bytes(self.h)

    def device_ptr(self, off=0):
        p = P()
        self.dev._check(lib().rk_arena_device_ptr(self.h, off, ctypes.byref(p)))
        return p.value

    def free(self):
        if self.h:
            self.dev._check(lib().rk_arena_free(self.h))
            self.h = None

    def begin(self):
        return Batch(self)


class Batch:
    """Recorded operations on an arena (internal/gpu Batch); the device is
    held from begin to submit. Reads land in numpy arrays on submit."""

    def __init__(self, arena):
        self.a, self.dev = arena, arena.dev
        h = P()
        self.dev._check(lib().rk_batch_begin(arena.h, ctypes.byref(h)))
        self.h = h
        self._keep = []

    def write(self, off, data):
        data = np.ascontiguousarray(data, dtype=np.float32)
        self._keep.append(data)
        return lib().rk_batch_write(self.h, off, _ptr(data), data.size)

    def read(self, off, n):
        dst = np.empty(n, np.float32)
        self._keep.append(dst)
        lib().rk_batch_read(self.h, off, _ptr(dst), n)
        return dst

    def matvecs(self, ms, out_offs, in_off):
        hs = (P * len(ms))(*[m.h for m in ms])
        offs = (I64 * len(ms))(*out_offs)
        return lib().rk_batch_matvecs(self.h, len(ms), hs, offs, in_off)

    def quantize(self, inp, n):
        return lib().rk_batch_quantize(self.h, inp, n)

    def quantize_fp8(self, inp, n):
        return lib().rk_batch_quantize_fp8(self.h, inp, n)

    def act_quant_inplace(self, off, n):
        return lib().rk_batch_act_quant_inplace(self.h, off, n)

    def fp4_quant_inplace(self, off, n, e4m3):
        return lib().rk_batch_fp4_quant_inplace(self.h, off, n, int(bool(e4m3)))

    def matvecs_batch(self, m, out, out_stride, inp, in_stride, n):
        """internal/gpu Batch.MatVecsBatch."""
        return lib().rk_batch_matvecs_batch(self.h, m.h, out, out_stride, inp, in_stride, n)

    def expert_matvecs(self, m, per_expert, ids, slots, inp, in_stride, div, out, out_stride):
        """internal/gpu Batch.ExpertMatVecs (ids: arena word of uint32 expert ids)."""
        return lib().rk_batch_expert_matvecs(self.h, m.h, per_expert, ids, slots, inp, in_stride, div, out,
                                             out_stride)

    def rmsnorm(self, vecs, inp, out, w, n, segs, stride, recip_n, eps):
        return lib().rk_batch_rmsnorm(self.h, vecs.h, inp, out, w, n, segs, stride, float(recip_n), float(eps))

    def addvec(self, vecs, out, v, n):
        return lib().rk_batch_addvec(self.h, vecs.h, out, v, n)

    def rope(self, q, k, q_dim, kv_dim, head_size, cos, sin):
        return lib().rk_batch_rope(self.h, q, k, q_dim, kv_dim, head_size, cos, sin)

    def copy(self, src, dst, n):
        return lib().rk_batch_copy(self.h, src, dst, n)

    def attention(self, q, keys, vals, att, att_stride, out, positions, heads, kv_heads, head_size, kv_dim, inv_sqrt):
        return lib().rk_batch_attention(self.h, q, keys, vals, att, att_stride, out, positions, heads, kv_heads,
                                        head_size, kv_dim, float(inv_sqrt))

    def residual(self, x, y, n, canonical):
        return lib().rk_batch_residual(self.h, x, y, n, int(canonical))

    def silumul(self, a, b, n):
        return lib().rk_batch_silumul(self.h, a, b, n)

    def submit(self):
        rc = lib().rk_batch_submit(self.h)
        self.h = None
        self._keep = []
        self.dev._check(rc)


class Device:
    """An opened GPU (internal/gpu Device)."""

    def __init__(self, index=0):
        h = P()
        rc = lib().rk_device_open(index, ctypes.byref(h))
        if rc != RK_OK:
            raise RKError(rc, lib().rk_last_error(None).decode())
        self.h = h

    def _check(self, rc):
        if rc != RK_OK:
            raise RKError(rc, lib().rk_last_error(self.h).decode())
        return rc

    def close(self):
        if self.h:
            lib().rk_device_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def used(self):
        return lib().rk_used_bytes(self.h)

    def upload(self, kind, rows, cols, w, scales=None):
        w = np.ascontiguousarray(w)
        sp = None
        if scales is not None:
            scales = np.ascontiguousarray(scales, dtype=np.float32)
            sp = _ptr(scales)
        h = P()
        self._check(lib().rk_matrix_upload(self.h, kind, rows, cols, _ptr(w), sp, ctypes.byref(h)))
        return Matrix(self, h, kind, rows, cols)

    def upload_mx(self, kind, rows, cols, w, e8m0):
        """An E4M3 (FP8) or packed E2M1 (FP4) matrix with its E8M0 scale
        bytes (internal/gpu Upload of Format{FP8 | FP4, E8M0})."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        e8m0 = np.ascontiguousarray(e8m0, dtype=np.uint8)
        h = P()
        self._check(lib().rk_matrix_upload_mx(self.h, kind, rows, cols, _ptr(w), _ptr(e8m0), ctypes.byref(h)))
        return Matrix(self, h, kind, rows, cols)

    def upload_mx_chunks(self, kind, rows, cols, w_chunks, s_chunks, align_rows=0):
        """Format{FP4Chunks, E8M0Chunks, AlignRows}: the codes and the scale
        bytes each given as a list of pieces read as one."""
        ws = [np.ascontiguousarray(c, dtype=np.uint8) for c in w_chunks]
        ss = [np.ascontiguousarray(c, dtype=np.uint8) for c in s_chunks]
        wp = (P * len(ws))(*[c.ctypes.data for c in ws])
        wl = (I64 * len(ws))(*[c.size for c in ws])
        sp = (P * len(ss))(*[c.ctypes.data for c in ss])
        sl = (I64 * len(ss))(*[c.size for c in ss])
        h = P()
        self._check(lib().rk_matrix_upload_mx_chunks(self.h, kind, rows, cols, len(ws), wp, wl, len(ss), sp, sl,
                                                     align_rows, ctypes.byref(h)))
        return Matrix(self, h, kind, rows, cols)

    def upload_q8(self, q, s, rows, cols):
        return self.upload(Q8, rows, cols, np.ascontiguousarray(q, dtype=np.int8), s)

    def upload_q4(self, q, s, rows, cols):
        return self.upload(Q4, rows, cols, np.ascontiguousarray(q, dtype=np.uint8), s)

    def matvecs(self, ms, x):
        """outs[i] = ms[i]·x with host buffers (internal/gpu MulVecs)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        outs = [np.empty(m.rows, np.float32) for m in ms]
        hs = (P * len(ms))(*[m.h for m in ms])
        ops = (P * len(ms))(*[o.ctypes.data for o in outs])
        self._check(lib().rk_matvecs(self.h, len(ms), hs, ops, _ptr(x), x.size))
        return outs

    def matvec(self, m, x):
        return self.matvecs([m], x)[0]

    def matmul_t(self, ms, x):
        """Batched products: x is [tokens][cols]; returns [tokens][rows_i] per
        matrix, each row what matvecs gives for that token alone."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        tokens, cols = x.shape
        outs = [np.empty((tokens, m.rows), np.float32) for m in ms]
        hs = (P * len(ms))(*[m.h for m in ms])
        ops = (P * len(ms))(*[_ptr(o) for o in outs])
        self._check(lib().rk_matmul_t(self.h, len(ms), hs, ops, _ptr(x), cols, tokens))
        return outs

    def matmul_t_device(self, ms, d_outs, d_x, cols, tokens, stream=None):
        """Enqueue batched products on device pointers (ints)."""
        hs = (P * len(ms))(*[m.h for m in ms])
        ops = (P * len(ms))(*d_outs)
        self._check(lib().rk_matmul_t_device(self.h, len(ms), hs, ops, P(d_x), cols, tokens,
                                             P(stream) if stream else None))

    def matmul_t_device_noalloc(self, ms, d_outs, d_x, cols, tokens, stream=None):
        """rk_matmul_t_device_noalloc: the same products with the quantized
        inputs in the library's static scratch (allocates nothing)."""
        hs = (P * len(ms))(*[m.h for m in ms])
        ops = (P * len(ms))(*d_outs)
        self._check(lib().rk_matmul_t_device_noalloc(self.h, len(ms), hs, ops, P(d_x), cols, tokens,
                                                     P(stream) if stream else None))

    def tensor_matmul(self, a, b, transposed=False):
        """rakkan_tensor_v1 matmul (b [k][n]) / matmul_t (b [n][k]) of 2-D
        float32 or int8 arrays; float32 or int32 result [m][n]."""
        if a.dtype != b.dtype or a.dtype not in (np.float32, np.int8):
            raise RKError(-1, "tensor matmul: f32 or i8 inputs of one type")
        a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
        m, k = a.shape
        n = b.shape[0] if transposed else b.shape[1]
        if (b.shape[1] if transposed else b.shape[0]) != k:
            raise RKError(-1, "tensor matmul: shapes differ")
        dt = TENSOR_F32 if a.dtype == np.float32 else TENSOR_I8
        c = np.empty((m, n), np.float32 if dt == TENSOR_F32 else np.int32)
        self._check(lib().rk_tensor_matmul(self.h, dt, int(bool(transposed)), m, k, n, _ptr(a), _ptr(b), _ptr(c)))
        return c

    def tensor_serve(self, fd, max_bytes=0):
        """The node side of the tensor broker (rk_tensor_serve): answers the
        worker's products arriving on descriptor fd until it closes its end."""
        self._check(lib().rk_tensor_serve(self.h, fd, max_bytes))

    def tensor_quantize(self, a, k):
        a = np.ascontiguousarray(a, np.float32)
        q = np.empty(a.shape, np.int8)
        self._check(lib().rk_tensor_quantize(self.h, _ptr(a), _ptr(q), a.size, k))
        return q

    def tensor_scale(self, a, k):
        a = np.ascontiguousarray(a)
        dt = {np.dtype(np.int32): TENSOR_I32, np.dtype(np.float32): TENSOR_F32, np.dtype(np.int8): TENSOR_I8}.get(
            a.dtype)
        if dt is None:
            raise RKError(-1, "tensor scale: f32 or i32 input")
        out = np.empty(a.shape, np.float32)
        self._check(lib().rk_tensor_scale(self.h, dt, _ptr(a), _ptr(out), a.size, k))
        return out

    def matvecs_device(self, ms, d_outs, d_x, cols, stream=None):
        """Enqueue products on device pointers (ints) on a HIP stream handle."""
        hs = (P * len(ms))(*[m.h for m in ms])
        ops = (P * len(ms))(*d_outs)
        self._check(lib().rk_matvecs_device(self.h, len(ms), hs, ops, P(d_x), cols, P(stream) if stream else None))

    def profile_start(self):
        self._check(lib().rk_profile_start(self.h))

    def profile_stop(self):
        """{kernel: (calls, total ms)} of the launches since profile_start."""
        n = I32()
        buf = (ProfileEntry * 64)()
        self._check(lib().rk_profile_stop(self.h, ctypes.cast(buf, P), 64, ctypes.byref(n)))
        return {buf[i].kernel.decode(): (buf[i].calls, buf[i].ms) for i in range(min(n.value, 64))}

    def launch_floor(self, nbytes, copies=8, launches=200):
        """(empty-kernel us, plain-read us) per launch, back to back: the floor
        under a launch that reads nbytes (rk_device_launch_floor)."""
        e, r = ctypes.c_float(), ctypes.c_float()
        self._check(lib().rk_device_launch_floor(self.h, nbytes, copies, launches, ctypes.byref(e), ctypes.byref(r)))
        return e.value, r.value

    def arena(self, words, staging_words):
        return Arena(self, words, staging_words)

    def upload_vectors(self, v):
        v = np.ascontiguousarray(v, dtype=np.float32)
        h = P()
        self._check(lib().rk_vectors_upload(self.h, _ptr(v), v.size, ctypes.byref(h)))
        return Vectors(self, h, v.size)

    def num_eval(self, fn, x):
        """The device's restatement of a package-num function on each of x."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self._check(lib().rk_num_eval(self.h, fn, _ptr(x), _ptr(out), x.size))
        return out

    def sample_logits(self, logits, temperature, state):
        """rk_sample_logits: Sampler.Sample of each row of logits [rows][vocab]
        with temperature[z] and generator state[z] (uint64, updated in place);
        the picked tokens."""
        lg = np.ascontiguousarray(logits, np.float32)
        lg = lg.reshape(1, -1) if lg.ndim == 1 else lg
        rows, vocab = lg.shape
        t = np.ascontiguousarray(np.broadcast_to(np.asarray(temperature, np.float32), (rows,)), np.float32)
        if state.dtype != np.uint64 or state.shape != (rows,) or not state.flags.c_contiguous:
            raise ValueError("state: a contiguous uint64 array of one state a row")
        out = np.empty(rows, np.int32)
        self._check(lib().rk_sample_logits(self.h, _ptr(lg), vocab, rows, _ptr(t), _ptr(state), _ptr(out)))
        return out

    def graph_begin(self):
        self._check(lib().rk_graph_begin(self.h))

    def graph_end(self):
        h = P()
        self._check(lib().rk_graph_end(self.h, ctypes.byref(h)))
        return Graph(self, h)


class Graph:
    """Recorded device work, replayed by launch (rk_graph_*)."""

    def __init__(self, dev, handle):
        self.dev, self.h = dev, handle

    def launch(self, times=1):
        self.dev._check(lib().rk_graph_launch(self.h, times))

    def launch_timed(self, times=1):
        """Replays `times` times and returns the device milliseconds from
        the first replay's start to the last one's end (stream events)."""
        ms = ctypes.c_float()
        self.dev._check(lib().rk_graph_launch_timed(self.h, times, ctypes.byref(ms)))
        return ms.value

    def free(self):
        if self.h:
            lib().rk_graph_free(self.h)
            self.h = None


class Moe:
    """A mixture-of-experts feed-forward on one device (rk_moe_*): a Q8
    router [experts][dim] and per expert Q8 W1/W3 [hidden][dim], W2
    [dim][hidden] (uploaded Matrix objects, kept by the caller)."""

    def __init__(self, dev, router, w1, w2, w3, topk):
        self.dev, self.topk = dev, topk
        self.dim = router.cols
        n = len(w1)
        arr = lambda ms: (P * n)(*[m.h for m in ms])  # noqa: E731
        h = P()
        dev._check(lib().rk_moe_new(dev.h, router.h, n, arr(w1), arr(w2), arr(w3), topk, ctypes.byref(h)))
        self.h = h

    def ffn(self, xn):
        """y [tokens][dim], selected experts and weights [tokens][topk]."""
        xn = np.ascontiguousarray(xn, np.float32).reshape(-1, self.dim)
        t = xn.shape[0]
        y = np.empty_like(xn)
        sel = np.empty((t, self.topk), np.int32)
        w = np.empty((t, self.topk), np.float32)
        self.dev._check(lib().rk_moe_ffn(self.h, _ptr(xn), t, _ptr(y), _ptr(sel), _ptr(w)))
        return y, sel, w

    def ffn_device(self, d_xn, tokens, d_y, stream=None):
        self.dev._check(lib().rk_moe_ffn_device(self.h, P(d_xn), tokens, P(d_y), P(stream) if stream else None))

    def bytes(self):
        return lib().rk_moe_bytes(self.h)

    def free(self):
        if self.h:
            self.dev._check(lib().rk_moe_free(self.h))
            self.h = None


class Stage:
    """A run of llama-family layers on one device (rk_stage_*; the
    reference's gpuStage, internal/llm/gpustage.go). `layers` is a list of
    dicts with the uploaded matrices (wq wk wv wo w1 w2 w3: Matrix) and the
    host vectors (rms_att rms_ffn, and bq bk bv / q_norm k_norm when the
    config has them). Constants the reference computes with package num
    (Recip32 of the widths) come from the device's own restatement."""

    def __init__(self, dev, dim, hidden, heads, kv_heads, ctx, layers, rope_cos, rope_sin, head_dim=0,
                 norm_eps=1e-5, qkv_bias=False, qk_norm=False, seqs=1):
        hs = head_dim if head_dim > 0 else dim // heads
        rd, rh = dev.num_eval(FN_RECIP32, np.array([dim, hs], np.float32))
        inv_sqrt = inv_sqrt_head(hs)
        self.dev, self.dim, self.ctx, self.hs, self.seqs = dev, dim, ctx, hs, seqs
        self.cfg = StageConfig(dim, hidden, heads, kv_heads, head_dim, ctx, int(qkv_bias), int(qk_norm),
                               float(np.float32(norm_eps)), float(rd), float(rh), float(inv_sqrt), seqs)
        self._keep = []
        arr = (StageLayer * len(layers))()
        for i, L in enumerate(layers):
            vals = {}
            moe = L.get("moe")  # a Moe in place of w1/w2/w3
            vals["moe"] = moe.h if moe is not None else None
            for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"):
                m = L.get(n)
                vals[n] = m.h if m is not None else None
            for n in ("rms_att", "rms_ffn", "bq", "bk", "bv", "q_norm", "k_norm"):
                v = L.get(n)
                if v is not None:
                    v = np.ascontiguousarray(v, np.float32)
                    self._keep.append(v)
                    vals[n] = v.ctypes.data
                else:
                    vals[n] = None
            arr[i] = StageLayer(**vals)
        cos = np.ascontiguousarray(rope_cos, np.float32)
        sin = np.ascontiguousarray(rope_sin, np.float32)
        h = P()
        dev._check(lib().rk_stage_new(dev.h, ctypes.byref(self.cfg), arr, len(layers), _ptr(cos), _ptr(sin),
                                      ctypes.byref(h)))
        self.h = h
        self.vocab = 0

    def forward(self, xs, pos):
        """Stage.ForwardMany: rows of xs (tokens x dim) at positions pos.., returned."""
        xs = np.array(xs, np.float32, copy=True).reshape(-1, self.dim)
        self.dev._check(lib().rk_stage_forward(self.h, _ptr(xs), pos, xs.shape[0]))
        return xs

    def set_head(self, embed, wcls, rms_final):
        rf = np.ascontiguousarray(rms_final, np.float32)
        self.dev._check(lib().rk_stage_set_head(self.h, embed.h, wcls.h, _ptr(rf)))
        self.vocab = wcls.rows

    def generate_start(self, prompt):
        p = np.ascontiguousarray(prompt, np.int32)
        self.dev._check(lib().rk_stage_generate_start(self.h, _ptr(p), len(p)))

    def generate_run(self, positions, want_logits=False):
        out = np.empty((positions, self.vocab), np.float32) if want_logits else None
        self.dev._check(lib().rk_stage_generate_run(self.h, positions, _ptr(out) if want_logits else None))
        return out

    def tokens(self, start, n):
        out = np.empty(n, np.int32)
        self.dev._check(lib().rk_stage_generate_tokens(self.h, start, n, _ptr(out)))
        return out

    def generate(self, prompt, steps):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(steps, np.int32)
        self.dev._check(lib().rk_stage_generate(self.h, _ptr(p), len(p), steps, _ptr(out)))
        return out

    def seqs_start(self, prompts):
        """rk_stage_seqs_start: one prompt (a list of token ids) per sequence."""
        lens = np.array([len(p) for p in prompts], np.int32)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int32) for p in prompts]), np.int32)
        self.dev._check(lib().rk_stage_seqs_start(self.h, _ptr(flat), _ptr(lens)))

    def seqs_run(self, steps, want_logits=False):
        """rk_stage_seqs_run: steps decode steps of every sequence; with
        want_logits, their logits [steps][seqs][vocab]."""
        out = np.empty((steps, self.seqs, self.vocab), np.float32) if want_logits else None
        self.dev._check(lib().rk_stage_seqs_run(self.h, steps, _ptr(out) if want_logits else None))
        return out

    def seqs_tokens(self, seq, start, n):
        out = np.empty(n, np.int32)
        self.dev._check(lib().rk_stage_seqs_tokens(self.h, seq, start, n, _ptr(out)))
        return out

    def sampler(self, temperature, seed, seq=0):
        """rk_stage_sampler: NewSampler(temperature, seed) for sequence seq
        (internal/llm/sample.go:11-16); temperature <= 0 is the greedy argmax."""
        self.dev._check(lib().rk_stage_sampler(self.h, seq, float(np.float32(temperature)), int(seed) & (2**64 - 1)))

    def moe_stats(self):
        """rk_stage_moe_stats: (experts selected summed over the batched MoE
        groupings, groupings) since the last call; the counters restart."""
        a, b = ctypes.c_int64(), ctypes.c_int64()
        self.dev._check(lib().rk_stage_moe_stats(self.h, ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    @property
    def bytes(self):
        return lib().rk_stage_bytes(self.h)

    def free(self):
        if self.h:
            lib().rk_stage_free(self.h)
            self.h = None
