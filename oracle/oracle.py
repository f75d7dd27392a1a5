"""ctypes front end of the CPU oracle (oracle/rk_oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module as the checker. The product (the HIP
backend under rakkan-mesh_amd/) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "librkoracle.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int32
F32 = ctypes.c_float
F64 = ctypes.c_double


def _declare(L):
    sig = {
        "rko_canonical": (F32, [F32]), "rko_pow2": (F32, [ctypes.c_int]), "rko_scale2": (F32, [F32, ctypes.c_int]),
        "rko_recip32": (F32, [F32]), "rko_rsqrt32": (F32, [F32]), "rko_exp32": (F32, [F32]),
        "rko_exp": (F64, [F64]), "rko_log": (F64, [F64]), "rko_log1p": (F64, [F64]), "rko_log32": (F32, [F32]),
        "rko_sincos": (None, [F64, P, P]), "rko_gomax": (F32, [F32, F32]),
        "rko_to_bf16": (ctypes.c_uint16, [F32]), "rko_bf16": (F32, [ctypes.c_uint16]),
        "rko_dot": (F32, [P, P, I64]), "rko_dot32": (F32, [P, P, I64]), "rko_dot_bf16": (F32, [P, P, I64]),
        "rko_matvec32": (None, [P, P, P, I64, I64]), "rko_matvec_bf16": (None, [P, P, P, I64, I64]),
        "rko_quantize8": (None, [P, I64, P, P]), "rko_quantize4": (None, [P, I64, P, P]),
        "rko_dequant8": (None, [P, P, P, I64]), "rko_dequant4": (None, [P, P, P, I64]),
        "rko_blocksums_q8": (None, [P, P, I64, P]), "rko_blocksums_q4": (None, [P, P, I64, P]),
        "rko_qrow": (F32, [P, P, P, I64]),
        "rko_matvec_q8": (None, [P, P, P, P, I64, I64]), "rko_matvec_q4": (None, [P, P, P, P, I64, I64]),
        "rko_matmul_q8": (None, [P, P, P, P, I64, I64, I64]), "rko_matmul_q4": (None, [P, P, P, P, I64, I64, I64]),
        "rko_matvec_q8_avx2_mt": (None, [P, P, P, P, I64, I64, ctypes.c_int]),
        "rko_matvec_q4_avx2_mt": (None, [P, P, P, P, I64, I64, ctypes.c_int]),
        "rko_have_avx2": (ctypes.c_int, []),
        "rko_pcg_seed": (None, [P, ctypes.c_uint64, ctypes.c_uint64]), "rko_pcg_uint64": (ctypes.c_uint64, [P]),
        "rko_rand_float64": (F64, [P]), "rko_rand_intn": (I64, [P, I64]),
        "rko_transcendental_words": (None, [P, I64]),
        "rko_matvec": (None, [P, P, P]), "rko_rope_table": (None, [P, I32, P, P]),
        "rko_rmsnorm": (None, [P, P, P, I64, F32]), "rko_softmax": (None, [P, I64]), "rko_silu": (F32, [F32]),
        "rko_inv_sqrt_head": (F32, [ctypes.c_int]),
        "rko_sampler_seed": (ctypes.c_uint64, [ctypes.c_uint64]), "rko_sampler_next": (F32, [P]),
        "rko_sample_probs": (None, [P, I64, F32, P]), "rko_sample": (I32, [P, I64, F32, P]),
        "rko_attention_head": (None, [P, P, P, I64, ctypes.c_int, ctypes.c_int, F32, P, P]),
        "rko_set_matvec_threads": (None, [ctypes.c_int]),
        "rko_forward": (None, [P, P, I32, P, P, P, P, I32, P, I32, P]),
        "rko_embed": (None, [P, P, I32, P]), "rko_logits": (None, [P, P, P, P, P]), "rko_argmax": (I32, [P, I64]),
        "rko_num_eval": (None, [ctypes.c_int, P, P, I64]),
        "rko_topk": (None, [P, I32, I32, P]),
        "rko_moe_ffn": (None, [P, P, P, P, I32, I32, P, P, P, P]),
        "rko_tensor_matmul_f32": (None, [P, P, P, I64, I64, I64, ctypes.c_int]),
        "rko_tensor_matmul_i8": (None, [P, P, P, I64, I64, I64, ctypes.c_int]),
        "rko_tensor_quantize": (None, [P, P, I64, F32]), "rko_tensor_scale_i32": (None, [P, P, I64, F32]),
        "rko_e4m3_value": (F64, [ctypes.c_uint8]), "rko_encode_e4m3_n": (None, [P, I64, P]),
        "rko_decode_e8m0": (F32, [ctypes.c_uint8]), "rko_decode_e2m1": (F32, [ctypes.c_uint8]),
        "rko_encode_e2m1": (ctypes.c_uint8, [F32]), "rko_pow2ceil": (F32, [F32]),
        "rko_act_fp8": (None, [P, I64, P, P]), "rko_act_quant_inplace": (None, [P, I64]),
        "rko_matvec_fp8": (None, [P, P, P, P, P, I64, I64, ctypes.c_int]),
        "rko_matvec_fp4": (None, [P, P, P, P, P, I64, I64, ctypes.c_int]),
        "rko_quantize_fp4": (None, [P, I64, ctypes.c_int, P, P]), "rko_dequant_fp4": (None, [P, I64, ctypes.c_int, P, P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def ptr(a):
    return a.ctypes.data_as(P)


# ---- scalar helpers -------------------------------------------------------

def recip32(x):
    return np.float32(lib().rko_recip32(np.float32(x)))


def rsqrt32(x):
    return np.float32(lib().rko_rsqrt32(np.float32(x)))


def exp32(x):
    return np.float32(lib().rko_exp32(np.float32(x)))


def num_eval(fn, x):
    """fn (0 Recip32, 1 Rsqrt32, 2 Exp32, 3 silu) of each of x."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().rko_num_eval(fn, ptr(x), ptr(out), x.size)
    return out


class Sampler:
    """internal/llm/sample.go Sampler: NewSampler(temperature, seed), then
    sample(logits) per generated token (the state advances one draw a
    sampled token)."""

    def __init__(self, temperature, seed):
        self.temperature = np.float32(temperature)
        self.state = ctypes.c_uint64(lib().rko_sampler_seed(ctypes.c_uint64(seed)))

    def next(self):
        return np.float32(lib().rko_sampler_next(ctypes.byref(self.state)))

    def sample(self, logits):
        v = np.ascontiguousarray(logits, np.float32)
        return int(lib().rko_sample(ptr(v), v.size, self.temperature, ctypes.byref(self.state)))


def sample_probs(logits, temperature):
    """p of Sample before the draw: softmax(logits / T) (sample.go:30-35)."""
    v = np.ascontiguousarray(logits, np.float32)
    p = np.empty_like(v)
    lib().rko_sample_probs(ptr(v), v.size, np.float32(temperature), ptr(p))
    return p


def argmax(v):
    """internal/llm/sample.go:45-53."""
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().rko_argmax(ptr(v), v.size))


# ---- vectors and matrices -------------------------------------------------

def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def quantize8(w):
    w = _c(w, np.float32).ravel()
    q = np.empty(w.size, np.int8)
    s = np.empty(w.size // 32, np.float32)
    lib().rko_quantize8(ptr(w), w.size, ptr(q), ptr(s))
    return q, s


def quantize4(w):
    w = _c(w, np.float32).ravel()
    q = np.empty(w.size // 2, np.uint8)
    s = np.empty(w.size // 32, np.float32)
    lib().rko_quantize4(ptr(w), w.size, ptr(q), ptr(s))
    return q, s


def matvec_q8(w, ws, x, rows, cols):
    w, ws, x = _c(w, np.int8), _c(ws, np.float32), _c(x, np.float32)
    out = np.empty(rows, np.float32)
    lib().rko_matvec_q8(ptr(out), ptr(w), ptr(ws), ptr(x), rows, cols)
    return out


def matvec_q4(w, ws, x, rows, cols):
    w, ws, x = _c(w, np.uint8), _c(ws, np.float32), _c(x, np.float32)
    out = np.empty(rows, np.float32)
    lib().rko_matvec_q4(ptr(out), ptr(w), ptr(ws), ptr(x), rows, cols)
    return out


def matmul_q8(w, ws, x, tokens, rows, cols):
    w, ws, x = _c(w, np.int8), _c(ws, np.float32), _c(x, np.float32)
    out = np.empty(tokens * rows, np.float32)
    lib().rko_matmul_q8(ptr(out), ptr(w), ptr(ws), ptr(x), tokens, rows, cols)
    return out.reshape(tokens, rows)


def matmul_q4(w, ws, x, tokens, rows, cols):
    w, ws, x = _c(w, np.uint8), _c(ws, np.float32), _c(x, np.float32)
    out = np.empty(tokens * rows, np.float32)
    lib().rko_matmul_q4(ptr(out), ptr(w), ptr(ws), ptr(x), tokens, rows, cols)
    return out.reshape(tokens, rows)


class matvec_threads:
    """Within the block, the model forward's Q8 / Q4 products (rko_matvec)
    run the AVX2 block sums on n threads (the same bits as the portable
    loops; for model-size checks)."""

    def __init__(self, n):
        self.n = n

    def __enter__(self):
        lib().rko_set_matvec_threads(self.n)
        return self

    def __exit__(self, *exc):
        lib().rko_set_matvec_threads(0)
        return False


def matvec_q8_avx2(w, ws, x, rows, cols, threads):
    w, ws, x = _c(w, np.int8), _c(ws, np.float32), _c(x, np.float32)
    out = np.empty(rows, np.float32)
    lib().rko_matvec_q8_avx2_mt(ptr(out), ptr(w), ptr(ws), ptr(x), rows, cols, threads)
    return out


def matvec_q4_avx2(w, ws, x, rows, cols, threads):
    w, ws, x = _c(w, np.uint8), _c(ws, np.float32), _c(x, np.float32)
    out = np.empty(rows, np.float32)
    lib().rko_matvec_q4_avx2_mt(ptr(out), ptr(w), ptr(ws), ptr(x), rows, cols, threads)
    return out


def matvec32(w, x, rows, cols):
    w, x = _c(w, np.float32), _c(x, np.float32)
    out = np.empty(rows, np.float32)
    lib().rko_matvec32(ptr(out), ptr(w), ptr(x), rows, cols)
    return out


def matvec_bf16(w, x, rows, cols):
    w, x = _c(w, np.uint16), _c(x, np.float32)
    out = np.empty(rows, np.float32)
    lib().rko_matvec_bf16(ptr(out), ptr(w), ptr(x), rows, cols)
    return out


def dot32(a, b):
    a, b = _c(a, np.float32), _c(b, np.float32)
    return np.float32(lib().rko_dot32(ptr(a), ptr(b), a.size))


def dot_bf16(w, x):
    w, x = _c(w, np.uint16), _c(x, np.float32)
    return np.float32(lib().rko_dot_bf16(ptr(w), ptr(x), w.size))


def to_bf16(v):
    v = _c(v, np.float32)
    return np.array([lib().rko_to_bf16(np.float32(t)) for t in v], np.uint16)


def rmsnorm(x, w, eps):
    x, w = _c(x, np.float32), _c(w, np.float32)
    out = np.empty_like(x)
    lib().rko_rmsnorm(ptr(out), ptr(x), ptr(w), x.size, np.float32(eps))
    return out


def softmax(x):
    x = _c(x, np.float32).copy()
    lib().rko_softmax(ptr(x), x.size)
    return x


def attention_head(q, keys, vals, inv_sqrt):
    """One head's attention (internal/llm/model.go:570-588): q [hs], keys and
    vals [positions][hs]; returns (weights [positions], out [hs])."""
    q, keys, vals = _c(q, np.float32), _c(keys, np.float32), _c(vals, np.float32)
    positions, hs = keys.shape
    att = np.empty(positions, np.float32)
    out = np.empty(hs, np.float32)
    lib().rko_attention_head(ptr(q), ptr(keys), ptr(vals), hs, hs, positions, np.float32(inv_sqrt), ptr(att),
                             ptr(out))
    return att, out


def topk(v, k):
    v = _c(v, np.float32)
    idx = np.empty(k, np.int32)
    lib().rko_topk(ptr(v), v.size, k, ptr(idx))
    return idx


def moe_ffn(router, w1, w2, w3, topk_n, xn):
    """The build's MoE feed-forward contract for one normed input (Mat
    objects of oracle.model): y, selected experts, their weights."""
    from .model import RkoMat
    n = len(w1)
    arr = lambda ms: (RkoMat * n)(*[m.ctype() for m in ms])  # noqa: E731
    a1, a2, a3 = arr(w1), arr(w2), arr(w3)
    rt = router.ctype()
    xn = _c(xn, np.float32)
    y = np.empty(router.cols, np.float32)
    sel = np.empty(topk_n, np.int32)
    w = np.empty(topk_n, np.float32)
    lib().rko_moe_ffn(ctypes.byref(rt), a1, a2, a3, n, topk_n, ptr(xn), ptr(y), ptr(sel), ptr(w))
    return y, sel, w


def tensor_matmul_f32(a, b, transposed):
    a, b = _c(a, np.float32), _c(b, np.float32)
    m, k = a.shape
    n = b.shape[0] if transposed else b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().rko_tensor_matmul_f32(ptr(a), ptr(b), ptr(c), m, k, n, int(transposed))
    return c


def tensor_matmul_i8(a, b, transposed):
    a, b = _c(a, np.int8), _c(b, np.int8)
    m, k = a.shape
    n = b.shape[0] if transposed else b.shape[1]
    c = np.empty((m, n), np.int32)
    lib().rko_tensor_matmul_i8(ptr(a), ptr(b), ptr(c), m, k, n, int(transposed))
    return c


def tensor_quantize(a, k):
    a = _c(a, np.float32)
    q = np.empty(a.shape, np.int8)
    lib().rko_tensor_quantize(ptr(a), ptr(q), a.size, np.float32(k))
    return q


def tensor_scale_i32(a, k):
    a = _c(a, np.int32)
    out = np.empty(a.shape, np.float32)
    lib().rko_tensor_scale_i32(ptr(a), ptr(out), a.size, np.float32(k))
    return out


def transcendental_digest(steps=100000):
    import hashlib
    buf = np.zeros(5 * steps, np.uint64)
    lib().rko_transcendental_words(ptr(buf), steps)
    return hashlib.sha256(buf.astype("<u8").tobytes()).hexdigest()


class PCG:
    """Go's math/rand/v2 PCG source with Float64 and IntN."""

    def __init__(self, s1, s2):
        self._st = (ctypes.c_uint64 * 2)()
        lib().rko_pcg_seed(ctypes.cast(self._st, P), s1, s2)

    def uint64(self):
        return lib().rko_pcg_uint64(ctypes.cast(self._st, P))

    def float64(self):
        return lib().rko_rand_float64(ctypes.cast(self._st, P))

    def intn(self, n):
        return lib().rko_rand_intn(ctypes.cast(self._st, P), n)


# ---- internal/num/mx.go: DeepSeek-V4.1 block-scaled formats ------------------

def e4m3_values():
    """The 256 E4M3 codes' values (float64; NaN for 0x7f and 0xff)."""
    L = lib()
    return np.array([L.rko_e4m3_value(c) for c in range(256)], np.float64)


def encode_e4m3(v):
    v = _c(v, np.float32).ravel()
    out = np.empty(v.size, np.uint8)
    lib().rko_encode_e4m3_n(ptr(v), v.size, ptr(out))
    return out


def act_fp8(x):
    """QuantizeActFP8: (E4M3 codes, float32 block scales)."""
    x = _c(x, np.float32).ravel()
    codes = np.empty(x.size, np.uint8)
    scales = np.empty(x.size // 32, np.float32)
    lib().rko_act_fp8(ptr(x), x.size, ptr(codes), ptr(scales))
    return codes, scales


def act_quant_inplace(x):
    x = _c(x, np.float32).ravel().copy()
    lib().rko_act_quant_inplace(ptr(x), x.size)
    return x


def matvec_fp8(w, ws, x, rows, cols, bf16=True):
    """MatVecFP8 (bf16) / MatVecFP8Unrounded of float32 input x."""
    codes, xs = act_fp8(x)
    w, ws = _c(w, np.uint8), _c(ws, np.uint8)
    out = np.empty(rows, np.float32)
    lib().rko_matvec_fp8(ptr(out), ptr(w), ptr(ws), ptr(codes), ptr(xs), rows, cols, int(bf16))
    return out


def matvec_fp4(w, ws, x, rows, cols, bf16=True):
    """MatVecFP4 (bf16) / MatVecFP4Unrounded of float32 input x."""
    codes, xs = act_fp8(x)
    w, ws = _c(w, np.uint8), _c(ws, np.uint8)
    out = np.empty(rows, np.float32)
    lib().rko_matvec_fp4(ptr(out), ptr(w), ptr(ws), ptr(codes), ptr(xs), rows, cols, int(bf16))
    return out


def quantize_fp4(x, e4m3):
    """QuantizeFP4: (packed codes, scale bytes); blocks of 16 with E4M3
    scales if e4m3, else of 32 with E8M0 scales."""
    x = _c(x, np.float32).ravel()
    blk = 16 if e4m3 else 32
    packed = np.zeros(x.size // 2, np.uint8)
    scales = np.empty(x.size // blk, np.uint8)
    lib().rko_quantize_fp4(ptr(x), x.size, int(e4m3), ptr(packed), ptr(scales))
    return packed, scales


def dequant_fp4(packed, scales, n, e4m3):
    packed, scales = _c(packed, np.uint8), _c(scales, np.uint8)
    x = np.empty(n, np.float32)
    lib().rko_dequant_fp4(ptr(x), n, int(e4m3), ptr(packed), ptr(scales))
    return x
