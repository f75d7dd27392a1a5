"""The reference's on-disk model formats, host side (numpy): llama2.c
checkpoints (internal/llm/model.go:702-800 ReadCheckpoint, Encode,
Quantize), model parts as a node stores them (internal/llm/shard.go:166-290
appendMatrix, EncodeLayer, LoadLayer, EncodeHead, LoadHead, LoadEmbed,
model.go:269-279, 390-400 matBytes, LayerBytes), and the weight quantizers
Quantize calls (internal/num/quant.go:25-126 QuantizeQ8 / QuantizeQ4,
recip.go:16-67 Recip32, matvec.go:22-29 ToBF16), restated with the same
float32 / float64 roundings so the codes are the reference's bit for bit.
Hugging Face models (internal/llm/hf.go: safetensors, float16/bfloat16
weights, the rotary row permutation, config.json's mapping) import to the
same parts.

`stage_from_checkpoint` uploads a quantized checkpoint's layers to a device
as an rkhip.Stage and its head, the way internal/llm moves layers to a GPU
(model.go:345-387)."""
from dataclasses import dataclass, field

import numpy as np

F32 = np.float32
_K_24_17 = np.array([0x3FB4B4B5], np.uint32).view(F32)[0]  # float32(24.0/17)   recip.go:54
_K_8_17 = np.array([0x3EF0F0F1], np.uint32).view(F32)[0]   # float32(8.0/17)    recip.go:54
_K_1_127 = np.array([0x3C010204], np.uint32).view(F32)[0]  # float32(1.0/127)   quant.go:42
_CANON_NAN = np.array([0x7FC00000], np.uint32).view(F32)[0]
QBLOCK = 32
DTYPES = ("", "f32", "bf16", "q8_0", "q4_0", "q4_m")


# --- internal/num: Recip32, ToBF16, QuantizeQ8, QuantizeQ4 ------------------

def _pow2(k):
    """2^k for integer k in [-126, 127] as float32, exactly (recip.go:16)."""
    return ((np.asarray(k, np.int64) + 127).astype(np.uint32) << 23).view(F32)


def _half_toward_zero(k):
    """Go's k/2 on ints (truncating)."""
    k = np.asarray(k, np.int64)
    return np.where(k >= 0, k // 2, -((-k) // 2))


def recip32(x):
    """internal/num/recip.go:36-67 Recip32, elementwise on float32."""
    x = np.asarray(x, F32)
    ax = np.abs(x)
    b = ax.view(np.uint32)
    finite = (ax == ax) & (ax != 0) & ~np.isinf(ax)
    sub = ((b >> 23) == 0) & finite
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        xs = np.where(sub, ax * _pow2(64), ax).astype(F32)
        bs = xs.view(np.uint32)
        e = np.where(sub, -64, 0) + (bs >> 23).astype(np.int64) - 127
        m = ((bs & 0x7FFFFF) | (127 << 23)).astype(np.uint32).view(F32)
        r = _K_24_17 - (_K_8_17 * m)
        for _ in range(3):
            r = r + (r * (F32(1) - (m * r)))
        ext = (e > 126) | (e < -127)
        k = -e
        k1 = _half_toward_zero(k)
        scaled = (r * _pow2(np.clip(k1, -126, 127))) * _pow2(np.clip(k - k1, -126, 127))
        plain = r * _pow2(np.clip(k, -126, 127))
        r = np.where(ext, scaled, plain).astype(F32)
    r = np.where(x < 0, -r, r).astype(F32)
    r = np.where(ax == 0, np.copysign(np.inf, x), r)
    r = np.where(np.isinf(ax), np.copysign(F32(0), x), r)
    return np.where(x != x, _CANON_NAN, r).astype(F32)


def to_bf16(f):
    """internal/num/matvec.go:22-29 ToBF16: round to nearest even bfloat16,
    NaNs stay NaN."""
    f = np.asarray(f, F32)
    b = f.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = f != f
    return np.where(nan, ((b >> 16).astype(np.uint16)) | 0x40, r).astype(np.uint16)


def _int8_of(r):
    """Go's int8(float64) of an already clamped value; NaN converts to 0
    (amd64's truncating conversion, then the low byte)."""
    return np.where(r == r, r, 0).astype(np.int8)


def quantize_q8(w):
    """internal/num/quant.go:24-53 QuantizeQ8: per 32-block d =
    amax·float32(1/127), q = int8(clamp(RoundToEven(float32(v·Recip32(d))),
    -127, 127)); zero codes when d is 0 or NaN."""
    w = np.ascontiguousarray(w, F32).ravel()
    blk = w.reshape(-1, QBLOCK)
    with np.errstate(invalid="ignore", over="ignore"):
        amax = np.max(np.abs(blk), axis=1)  # Go max: NaN if any is NaN
        d = (amax * _K_1_127).astype(F32)
        skip = (d == 0) | (d != d)
        idv = recip32(np.where(skip, F32(1), d))
        p = (blk * idv[:, None]).astype(F32)
        r = np.clip(np.rint(p.astype(np.float64)), -127, 127)
    q = _int8_of(r)
    q[skip] = 0
    return q.ravel(), d


def _quant4(blk, d):
    """internal/num/quant.go:120-126 quant4."""
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        idv = np.where(d != 0, F32(1) / np.where(d != 0, d, F32(1)), F32(0)).astype(F32)
        p = (blk * idv[:, None]).astype(F32)
        r = np.clip(np.rint(p.astype(np.float64)), -8, 7)
    return _int8_of(r)


def quantize_q4(w):
    """internal/num/quant.go:62-117 QuantizeQ4: per block, from scales that
    put the largest weight at -8, -7.5, -7, 7, 7.5 and 6.5, three rounds of
    rounding and the least-squares scale, the smallest squared error kept;
    float64 sums in element order, every product rounded as the reference
    rounds it."""
    w = np.ascontiguousarray(w, F32).ravel()
    blk = w.reshape(-1, QBLOCK)
    nb = blk.shape[0]
    amax = np.zeros(nb, F32)
    peak = np.zeros(nb, F32)
    a = np.abs(blk)
    for j in range(QBLOCK):  # the first largest magnitude wins (strict >)
        up = a[:, j] > amax
        amax = np.where(up, a[:, j], amax)
        peak = np.where(up, blk[:, j], peak)
    valid = (amax > 0) & (amax == amax)
    best_err = np.full(nb, np.inf)
    best_d = np.zeros(nb, F32)
    best = np.zeros((nb, QBLOCK), np.int8)
    b64 = blk.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        for div in (-8.0, -7.5, -7.0, 7.0, 7.5, 6.5):
            d = (peak / F32(div)).astype(F32)
            live = valid.copy()
            for _ in range(3):
                vals = _quant4(blk, d)
                v64 = vals.astype(np.float64)
                wq = np.zeros(nb)
                qq = np.zeros(nb)
                for j in range(QBLOCK):
                    wq = wq + b64[:, j] * v64[:, j]
                    qq = qq + v64[:, j] * v64[:, j]
                live = live & (qq != 0)
                d = np.where(live, (wq / np.where(qq != 0, qq, 1.0)).astype(F32), d).astype(F32)
            vals = _quant4(blk, d)
            deq = (vals.astype(F32) * d[:, None]).astype(F32).astype(np.float64)
            e = np.zeros(nb)
            for j in range(QBLOCK):
                diff = b64[:, j] - deq[:, j]
                e = e + diff * diff
            better = valid & (e < best_err)
            best_err = np.where(better, e, best_err)
            best_d = np.where(better, d, best_d).astype(F32)
            best = np.where(better[:, None], vals, best)
    lo = (best[:, :16].astype(np.int16) + 8).astype(np.uint8)
    hi = (best[:, 16:].astype(np.int16) + 8).astype(np.uint8)
    return (lo | (hi << 4)).astype(np.uint8).ravel(), best_d


# --- internal/llm: Config, Matrix, Layer, Head, Checkpoint --------------------

@dataclass
class Config:
    """internal/llm/model.go:37-66 Config."""
    dim: int
    hidden_dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    vocab_size: int
    seq_len: int
    shared_classifier: bool = False
    head_dim: int = 0
    rope_theta: float = 0.0
    norm_eps: float = 0.0
    qkv_bias: bool = False
    qk_norm: bool = False
    dtype: str = ""

    def head_size(self):
        return self.head_dim if self.head_dim > 0 else self.dim // self.n_heads

    def q_dim(self):
        return self.n_heads * self.head_size()

    def kv_dim(self):
        return self.n_kv_heads * self.head_size()

    def quantized(self):
        return self.dtype in ("q8_0", "q4_0", "q4_m")

    def embed_type(self):
        """model.go:96-101: q4_0 and q4_m keep the embedding and classifier in q8_0."""
        return "q8_0" if self.dtype in ("q4_0", "q4_m") else self.dtype

    def mat_type(self, sensitive):
        """model.go:105-113: q4_m keeps the value and down projections in q8_0."""
        if self.dtype != "q4_m":
            return self.dtype
        return "q8_0" if sensitive else "q4_0"

    def validate(self):
        """model.go:115-133 validate; raises ValueError with its messages."""
        c = self
        if min(c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.vocab_size, c.seq_len) <= 0 or c.head_dim < 0:
            raise ValueError("non-positive dimension")
        if (c.head_dim == 0 and c.dim % c.n_heads != 0) or c.n_heads % c.n_kv_heads != 0 or c.head_size() % 2 != 0:
            raise ValueError("heads do not divide the model dimension evenly")
        if (c.dim > 1 << 16 or c.hidden_dim > 1 << 18 or c.n_layers > 1024 or c.vocab_size > 1 << 20
                or c.seq_len > 1 << 20 or c.head_size() > 1024 or c.n_heads > 1024):
            raise ValueError("dimensions out of range")
        if c.dtype not in DTYPES:
            raise ValueError(f'unknown weight type "{c.dtype}"')
        if c.quantized() and (c.dim % QBLOCK or c.q_dim() % QBLOCK or c.hidden_dim % QBLOCK):
            raise ValueError(f"{c.dtype} needs widths that are multiples of {QBLOCK}")
        if c.rope_theta < 0 or c.norm_eps < 0 or c.norm_eps > 1:
            raise ValueError("rope base or norm epsilon out of range")


@dataclass
class Matrix:
    """model.go:136-146 Matrix: exactly one of f32, bf16, q8 (+ scales), q4 (+ scales)."""
    f32: np.ndarray = None
    bf16: np.ndarray = None
    q8: np.ndarray = None
    q4: np.ndarray = None
    scales: np.ndarray = None

    def floats(self):
        if self.f32 is not None:
            return self.f32
        if self.bf16 is not None:
            return (self.bf16.astype(np.uint32) << 16).view(F32)
        raise ValueError("a quantized matrix has no float form here")

    def convert(self, dtype):
        """model.go:247-266 convert."""
        if dtype == "q8_0":
            q, s = quantize_q8(self.floats())
            return Matrix(q8=q, scales=s)
        if dtype == "q4_0":
            q, s = quantize_q4(self.floats())
            return Matrix(q4=q, scales=s)
        if dtype == "bf16":
            return self if self.bf16 is not None else Matrix(bf16=to_bf16(self.f32))
        return Matrix(f32=self.floats())


@dataclass
class Layer:
    """model.go:281-294 Layer."""
    rms_att: np.ndarray = None
    wq: Matrix = None
    wk: Matrix = None
    wv: Matrix = None
    wo: Matrix = None
    bq: np.ndarray = None
    bk: np.ndarray = None
    bv: np.ndarray = None
    q_norm: np.ndarray = None
    k_norm: np.ndarray = None
    rms_ffn: np.ndarray = None
    w1: Matrix = None
    w2: Matrix = None
    w3: Matrix = None


def tensors(c: Config):
    """model.go:328-343 Layer.tensors: (name, is_matrix, size, cols, dtype)
    in storage order."""
    d, q, kv, h, hs = c.dim, c.q_dim(), c.kv_dim(), c.hidden_dim, c.head_size()
    m, s = c.mat_type(False), c.mat_type(True)
    t = [("rms_att", False, d, 0, ""), ("wq", True, q * d, d, m), ("wk", True, kv * d, d, m),
         ("wv", True, kv * d, d, s), ("wo", True, d * q, q, m), ("rms_ffn", False, d, 0, ""),
         ("w1", True, h * d, d, m), ("w2", True, d * h, h, s), ("w3", True, h * d, d, m)]
    if c.qkv_bias:
        t += [("bq", False, q, 0, ""), ("bk", False, kv, 0, ""), ("bv", False, kv, 0, "")]
    if c.qk_norm:
        t += [("q_norm", False, hs, 0, ""), ("k_norm", False, hs, 0, "")]
    return t


@dataclass
class Head:
    """model.go Head: the final norm and the classifier."""
    rms_final: np.ndarray = None
    wcls: Matrix = None


@dataclass
class Checkpoint:
    """model.go:705-710 Checkpoint."""
    config: Config
    embed: Matrix
    layers: list = field(default_factory=list)
    head: Head = None

    def encode(self):
        """model.go:773-800 Encode (float32 only; the legacy rotary tables as zeros)."""
        c = self.config
        vocab = c.vocab_size if c.shared_classifier else -c.vocab_size
        parts = [np.array([c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, vocab, c.seq_len],
                          np.int32).tobytes(), _f32(self.embed.f32)]
        for name, is_mat, _, _, _ in tensors(c):
            for ly in self.layers:
                v = getattr(ly, name)
                parts.append(_f32(v.f32 if is_mat else v))
        parts.append(_f32(self.head.rms_final))
        parts.append(bytes(4 * c.seq_len * c.head_size()))
        if not c.shared_classifier:
            parts.append(_f32(self.head.wcls.f32))
        return b"".join(parts)

    def quantize(self, dtype):
        """model.go:678-700 Quantize: the matrices to dtype ("bf16", "q8_0",
        "q4_0" or "q4_m"); the embedding and classifier to embed_type."""
        c = Config(**{**self.config.__dict__, "dtype": dtype})
        c.validate()
        for ly in self.layers:
            for name, is_mat, _, _, dt in tensors(c):
                if is_mat:
                    setattr(ly, name, getattr(ly, name).convert(dt))
        self.embed = self.embed.convert(c.embed_type())
        if c.shared_classifier:
            self.head.wcls = self.embed
        else:
            self.head.wcls = self.head.wcls.convert(c.embed_type())
        self.config = c


def _f32(v):
    return np.ascontiguousarray(v, "<f4").tobytes()


def read_checkpoint(data: bytes) -> Checkpoint:
    """model.go:721-769 ReadCheckpoint: seven int32s (dim, hidden_dim,
    n_layers, n_heads, n_kv_heads, vocab_size, seq_len; a negative
    vocab_size means a separate classifier), then the weights, grouped by
    tensor across layers. Raises ValueError with the reference's messages."""
    if len(data) < 28:
        raise ValueError("checkpoint too short")
    h = [int(v) for v in np.frombuffer(data[:28], "<i4")]
    c = Config(h[0], h[1], h[2], h[3], h[4], h[5], h[6], shared_classifier=h[5] > 0)
    if c.vocab_size < 0:
        c.vocab_size = -c.vocab_size
    try:
        c.validate()
    except ValueError as e:
        raise ValueError(f"checkpoint: {e}") from None
    off = 28

    def take(n):
        nonlocal off
        if n < 0 or off + 4 * n > len(data):
            raise ValueError("checkpoint truncated")
        v = np.frombuffer(data, "<f4", n, off).astype(F32)
        off += 4 * n
        return v

    ck = Checkpoint(c, Matrix(f32=take(c.vocab_size * c.dim)), [Layer() for _ in range(c.n_layers)], Head())
    for name, is_mat, size, _, _ in tensors(c):
        for ly in ck.layers:
            v = take(size)
            setattr(ly, name, Matrix(f32=v) if is_mat else v)
    ck.head.rms_final = take(c.dim)
    take(c.seq_len * c.head_size())  # legacy rotary tables, unused (NewRope computes them)
    ck.head.wcls = ck.embed if c.shared_classifier else Matrix(f32=take(c.vocab_size * c.dim))
    return ck


# --- model parts (internal/llm/shard.go) -------------------------------------

def mat_bytes(dtype, n):
    """model.go:269-279 matBytes."""
    if dtype == "bf16":
        return 2 * n
    if dtype == "q8_0":
        return n + (n // QBLOCK) * 4
    if dtype == "q4_0":
        return n // 2 + (n // QBLOCK) * 4
    return 4 * n


def layer_bytes(c: Config):
    """model.go:390-400 LayerBytes."""
    return sum(mat_bytes(dt, size) if is_mat else 4 * size for _, is_mat, size, _, dt in tensors(c))


def embed_bytes(c: Config):
    """shard.go EmbedBytes."""
    return mat_bytes(c.embed_type(), c.vocab_size * c.dim)


def append_matrix(m: Matrix):
    """shard.go:166-186 appendMatrix: float32, bfloat16, or quantized as the
    scales (float32) then the values."""
    if m.q8 is not None:
        return _f32(m.scales) + np.ascontiguousarray(m.q8, np.int8).tobytes()
    if m.q4 is not None:
        return _f32(m.scales) + np.ascontiguousarray(m.q4, np.uint8).tobytes()
    if m.bf16 is not None:
        return np.ascontiguousarray(m.bf16, "<u2").tobytes()
    return _f32(m.f32)


class _Decoder:
    """shard.go:188-249 decoder."""

    def __init__(self, data):
        self.data, self.at = data, 0

    def take(self, n):
        if n < 0 or self.at + n > len(self.data):
            raise ValueError("model part has the wrong size")
        b = self.data[self.at:self.at + n]
        self.at += n
        return b

    def vec(self, n):
        return np.frombuffer(self.take(4 * n), "<f4").astype(F32)

    def mat(self, n, dtype):
        if dtype == "q8_0":
            s = self.vec(n // QBLOCK)
            return Matrix(q8=np.frombuffer(self.take(n), np.int8).copy(), scales=s)
        if dtype == "q4_0":
            s = self.vec(n // QBLOCK)
            return Matrix(q4=np.frombuffer(self.take(n // 2), np.uint8).copy(), scales=s)
        if dtype == "bf16":
            return Matrix(bf16=np.frombuffer(self.take(2 * n), "<u2").astype(np.uint16))
        return Matrix(f32=self.vec(n))

    def done(self):
        if self.at != len(self.data):
            raise ValueError("model part has the wrong size")


def encode_layer(c: Config, ly: Layer):
    """shard.go:251-262 EncodeLayer."""
    return b"".join(append_matrix(getattr(ly, n)) if is_mat else _f32(getattr(ly, n))
                    for n, is_mat, _, _, _ in tensors(c))


def load_layer(c: Config, data: bytes):
    """shard.go:264-276 LoadLayer."""
    d, ly = _Decoder(data), Layer()
    for n, is_mat, size, _, dt in tensors(c):
        setattr(ly, n, d.mat(size, dt) if is_mat else d.vec(size))
    d.done()
    return ly


def encode_head(c: Config, h: Head):
    """shard.go:278-285 EncodeHead: a shared classifier is not stored."""
    b = _f32(h.rms_final)
    return b if c.shared_classifier else b + append_matrix(h.wcls)


def load_embed(c: Config, data: bytes):
    """shard.go LoadEmbed."""
    d = _Decoder(data)
    m = d.mat(c.vocab_size * c.dim, c.embed_type())
    d.done()
    return m


def load_head(c: Config, data: bytes, embed: Matrix):
    """shard.go LoadHead: a shared classifier is the embedding table."""
    d = _Decoder(data)
    h = Head(rms_final=d.vec(c.dim), wcls=embed)
    if not c.shared_classifier:
        h.wcls = d.mat(c.vocab_size * c.dim, c.embed_type())
    d.done()
    return h


# --- Hugging Face models (internal/llm/hf.go) ---------------------------------

HF_MODEL_TYPES = ("llama", "mistral", "qwen2", "qwen3")
_ST_HEADER_MAX = 100 << 20  # hf.go:84


class _Bytes:
    """A file read in pieces (hf.go:39-43 SizedReaderAt) over bytes in memory."""

    def __init__(self, b):
        self.b = memoryview(b)
        self.size = len(b)

    def read_at(self, off, n):
        return bytes(self.b[off:off + n])


class _File:
    """A file read in pieces from disk, one tensor at a time."""

    def __init__(self, path):
        self.path = path
        import os
        self.size = os.path.getsize(path)

    def read_at(self, off, n):
        with open(self.path, "rb") as f:
            f.seek(off)
            b = f.read(n)
        if len(b) != n:
            raise ValueError("unexpected EOF")
        return b


def _reader(f):
    if isinstance(f, (bytes, bytearray, memoryview)):
        return _Bytes(f)
    if isinstance(f, str):
        return _File(f)
    return f  # anything with read_at(off, n) and size


@dataclass
class STTensor:
    """hf.go:67-75 stTensor: a tensor's type, shape and byte range in a
    safetensors file."""
    dtype: str
    shape: list
    offsets: tuple
    file: object = None
    base: int = 0

    def elems(self):
        n = 1
        for d in self.shape:
            n *= d
        return n

    def raw(self, name, want):
        """hf.go:117-137 raw: the tensor's bytes, checking its type and
        element count. Returns (bytes, element size)."""
        size = {"BF16": 2, "F16": 2, "F32": 4}.get(self.dtype)
        if size is None:
            raise ValueError(f"tensor {name}: type {self.dtype} not supported")
        if self.elems() != want or want * size != self.offsets[1] - self.offsets[0]:
            raise ValueError(f"tensor {name}: shape {self.shape}, want {want} elements")
        return self.file.read_at(self.base + self.offsets[0], want * size), size


def read_safetensors(f, into: dict):
    """hf.go:77-115 readSafetensors: an 8-byte little-endian header size, a
    JSON header naming each tensor's type, shape and byte range, then the
    data. Adds the file's tensors to `into` (name -> STTensor); f is a path,
    bytes, or an object with read_at(off, n) and size. The header is parsed
    as JSON only; no tensor data is read here."""
    import json

    r = _reader(f)
    if r.size < 8:
        raise ValueError("safetensors: unexpected EOF")
    n = int(np.frombuffer(r.read_at(0, 8), "<u8")[0])
    if n > _ST_HEADER_MAX or n + 8 > r.size:
        raise ValueError(f"safetensors: header of {n} bytes")
    try:
        h = json.loads(r.read_at(8, n))
    except ValueError as e:
        raise ValueError(f"safetensors header: {e}") from None
    if not isinstance(h, dict):
        raise ValueError("safetensors header: not an object")
    base = 8 + n
    for name, v in h.items():
        if name == "__metadata__":
            continue
        try:
            off = v.get("data_offsets") or [0, 0]
            t = STTensor(str(v.get("dtype", "")), [int(d) for d in v.get("shape") or []],
                         (int(off[0]), int(off[1])), r, base)
        except (AttributeError, TypeError, ValueError, IndexError) as e:
            raise ValueError(f"safetensors tensor {name}: {e}") from None
        if t.offsets[0] < 0 or t.offsets[1] < t.offsets[0] or base + t.offsets[1] > r.size:
            raise ValueError(f"safetensors tensor {name}: data outside the file")
        if name in into:
            raise ValueError(f"safetensors: tensor {name} in two files")
        into[name] = t


def f16_to_f32(h):
    """hf.go:139-155 f16ToF32 over an array of IEEE half bit patterns:
    exact, subnormals normalized, infinities and NaNs keep their payload
    (shifted up 13 bits, the quiet bit as it was)."""
    h = np.asarray(h, np.uint16).astype(np.uint32)
    sign = (h >> 15) << 31
    exp = (h >> 10) & 0x1F
    frac = h & 0x3FF
    out = sign | ((exp + (127 - 15)) << 23) | (frac << 13)  # normal numbers
    out = np.where(exp == 0x1F, sign | 0x7F800000 | (frac << 13), out)
    # subnormals: shift the fraction up until its leading bit reaches 0x400
    sub = (exp == 0) & (frac != 0)
    e = np.full(h.shape, -14, np.int64)
    f = frac.copy()
    for _ in range(10):
        m = sub & ((f & 0x400) == 0)
        f = np.where(m, f << 1, f)
        e = np.where(m, e - 1, e)
    out = np.where(sub, sign | ((e + 127).astype(np.uint32) << 23) | ((f & 0x3FF) << 13), out)
    out = np.where((exp == 0) & (frac == 0), sign, out)
    return out.astype(np.uint32).view(F32)


def permute_rows(w, rows, head):
    """hf.go:235-249 permuteRows: each head's rows from Hugging Face's
    rotary layout (dimension j turns with j + head/2) to the engine's
    (adjacent pairs turn together): row 2j takes row j, row 2j+1 takes row
    j + head/2. Returns the permuted array (w is not changed)."""
    w = np.asarray(w)
    n = w.size // rows
    half = head // 2
    src = np.empty(head, np.int64)
    src[0::2] = np.arange(half)
    src[1::2] = np.arange(half) + half
    blocks = w.reshape(rows // head, head, n)
    return np.ascontiguousarray(blocks[:, src, :]).reshape(w.shape)


def permute_vec(v, head):
    """hf.go:251 permuteVec."""
    return permute_rows(v, len(v), head)


def _cfg_int(hc, key):
    v = hc.get(key)
    if v is None:
        return 0
    if isinstance(v, bool) or not isinstance(v, (int, float)) or (isinstance(v, float) and not v.is_integer()):
        raise ValueError(f"config.json: {key} is not an integer")
    return int(v)


def _cfg_float(hc, key):
    v = hc.get(key)
    if v is None:
        return 0.0
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        raise ValueError(f"config.json: {key} is not a number")
    return float(v)


def hf_config_of(hc: dict, weights: dict) -> Config:
    """hf.go:253-307 hfConfigOf: config.json (parsed) and the tensor table
    to a Config, refusing what the engine would run differently from the
    model's definition. Raises ValueError with the reference's messages."""
    import json

    mt = hc.get("model_type") or ""
    if mt not in HF_MODEL_TYPES:
        raise ValueError(f'model type "{mt}" is not supported (llama, mistral, qwen2, qwen3)')
    act = hc.get("hidden_act") or ""
    if act not in ("", "silu"):
        raise ValueError(f'activation "{act}" is not supported')
    if hc.get("rope_scaling") is not None:
        raise ValueError(f"rope scaling {json.dumps(hc['rope_scaling'], separators=(',', ':'))} is not supported")
    c = Config(dim=_cfg_int(hc, "hidden_size"), hidden_dim=_cfg_int(hc, "intermediate_size"),
               n_layers=_cfg_int(hc, "num_hidden_layers"), n_heads=_cfg_int(hc, "num_attention_heads"),
               n_kv_heads=_cfg_int(hc, "num_key_value_heads"), vocab_size=_cfg_int(hc, "vocab_size"),
               seq_len=_cfg_int(hc, "max_position_embeddings"), rope_theta=_cfg_float(hc, "rope_theta"),
               norm_eps=_cfg_float(hc, "rms_norm_eps"), shared_classifier=bool(hc.get("tie_word_embeddings")))
    if c.n_kv_heads == 0:
        c.n_kv_heads = c.n_heads
    hd = _cfg_int(hc, "head_dim")
    if hd > 0 and (c.n_heads == 0 or hd != c.dim // c.n_heads):
        c.head_dim = hd
    if c.rope_theta == 0:
        c.rope_theta = 10000.0
    if c.norm_eps == 0:
        c.norm_eps = 1e-6
    # within a sliding window attention is ordinary attention: the context
    # is capped to the window rather than masked
    win, use = hc.get("sliding_window"), hc.get("use_sliding_window")
    if isinstance(win, int) and not isinstance(win, bool) and 0 < win < c.seq_len and (use is None or use):
        c.seq_len = win
    if "lm_head.weight" not in weights:
        c.shared_classifier = True
    c.qkv_bias = "model.layers.0.self_attn.q_proj.bias" in weights
    c.qk_norm = "model.layers.0.self_attn.q_norm.weight" in weights
    et = weights.get("model.embed_tokens.weight")
    c.dtype = "bf16" if et is not None and et.dtype == "BF16" else "f32"
    if "model.layers.0.self_attn.o_proj.bias" in weights:
        raise ValueError("output projection biases are not supported")
    c.validate()
    return c


class HFModel:
    """hf.go:158-233 hfModel: tensors read by name in the target config's
    types, one at a time."""

    def __init__(self, c: Config, tensors_: dict):
        self.c, self.tensors = c, tensors_

    def _get(self, name):
        t = self.tensors.get(name)
        if t is None:
            raise ValueError(f"tensor {name} missing")
        return t

    def vec(self, name, n):
        """hf.go:164-187 vec: float32, bfloat16 or float16 to float32."""
        t = self._get(name)
        b, size = t.raw(name, n)
        if size == 4:
            return np.frombuffer(b, "<f4").astype(F32)
        u = np.frombuffer(b, "<u2").astype(np.uint16)
        if t.dtype == "BF16":
            return (u.astype(np.uint32) << 16).view(F32)
        return f16_to_f32(u)

    def mat(self, name, n, dtype):
        """hf.go:189-232 mat: a matrix stored as dtype; bfloat16 tensors
        stay as they are for a bfloat16 target, other types round to it."""
        if dtype in ("q8_0", "q4_0"):
            return Matrix(f32=self.vec(name, n)).convert(dtype)
        if dtype == "bf16":
            t = self._get(name)
            if t.dtype == "BF16":
                b, _ = t.raw(name, n)
                return Matrix(bf16=np.frombuffer(b, "<u2").astype(np.uint16))
            return Matrix(bf16=to_bf16(self.vec(name, n)))
        return Matrix(f32=self.vec(name, n))

    def layer(self, i):
        """hf.go:382-440 layer: query and key rows (and their biases and
        head norms) permuted to the engine's rotary layout before they are
        converted to the stored type."""
        c = self.c
        p = f"model.layers.{i}."
        d, q, kv, h, hs = c.dim, c.q_dim(), c.kv_dim(), c.hidden_dim, c.head_size()
        ly = Layer()
        ly.rms_att = self.vec(p + "input_layernorm.weight", d)
        wq = self.mat(p + "self_attn.q_proj.weight", q * d, "f32")
        wk = self.mat(p + "self_attn.k_proj.weight", kv * d, "f32")
        ly.wv = self.mat(p + "self_attn.v_proj.weight", kv * d, c.mat_type(True))
        ly.wo = self.mat(p + "self_attn.o_proj.weight", d * q, c.mat_type(False))
        ly.rms_ffn = self.vec(p + "post_attention_layernorm.weight", d)
        ly.w1 = self.mat(p + "mlp.gate_proj.weight", h * d, c.mat_type(False))
        ly.w2 = self.mat(p + "mlp.down_proj.weight", d * h, c.mat_type(True))
        ly.w3 = self.mat(p + "mlp.up_proj.weight", h * d, c.mat_type(False))
        if c.qkv_bias:
            ly.bq = self.vec(p + "self_attn.q_proj.bias", q)
            ly.bk = self.vec(p + "self_attn.k_proj.bias", kv)
            ly.bv = self.vec(p + "self_attn.v_proj.bias", kv)
        if c.qk_norm:
            ly.q_norm = self.vec(p + "self_attn.q_norm.weight", hs)
            ly.k_norm = self.vec(p + "self_attn.k_norm.weight", hs)
        ly.wq = Matrix(f32=permute_rows(wq.f32, q, hs)).convert(c.mat_type(False))
        ly.wk = Matrix(f32=permute_rows(wk.f32, kv, hs)).convert(c.mat_type(False))
        if c.qkv_bias:
            ly.bq, ly.bk = permute_vec(ly.bq, hs), permute_vec(ly.bk, hs)
        if c.qk_norm:
            ly.q_norm, ly.k_norm = permute_vec(ly.q_norm, hs), permute_vec(ly.k_norm, hs)
        return ly


def import_hf(config_json, weights, quant="") -> Checkpoint:
    """hf.go:310-380 ImportHF, without the store: config.json (bytes or
    str) and the safetensors files (paths, bytes, or readers; all shards in
    any order) to a Checkpoint of the model's parts in their stored types
    (encode_layer / encode_head / append_matrix give a node's bytes).
    quant, if set, stores the matrices as "bf16", "q8_0", "q4_0" or "q4_m"
    instead of the type they come in. The tokenizer, stop tokens and chat
    format (hf.go:331-335, 442-483) are not read here."""
    import json

    try:
        hc = json.loads(config_json)
    except ValueError as e:
        raise ValueError(f"config.json: {e}") from None
    if not isinstance(hc, dict):
        raise ValueError("config.json: not an object")
    ts = {}
    for f in weights:
        read_safetensors(f, ts)
    c = hf_config_of(hc, ts)
    if quant:
        c.dtype = quant
        c.validate()
    hm = HFModel(c, ts)
    embed = hm.mat("model.embed_tokens.weight", c.vocab_size * c.dim, c.embed_type())
    head = Head(rms_final=hm.vec("model.norm.weight", c.dim), wcls=embed)
    if not c.shared_classifier:
        head.wcls = hm.mat("lm_head.weight", c.vocab_size * c.dim, c.embed_type())
    return Checkpoint(c, embed, [hm.layer(i) for i in range(c.n_layers)], head)


# --- onto a device -----------------------------------------------------------

def upload_matrix(dev, m: Matrix, rows, cols):
    """One matrix through rk_matrix_upload in its own format."""
    from . import BF16, F32 as KF32, Q4, Q8

    if m.q8 is not None:
        return dev.upload(Q8, rows, cols, m.q8, m.scales)
    if m.q4 is not None:
        return dev.upload(Q4, rows, cols, m.q4, m.scales)
    if m.bf16 is not None:
        return dev.upload(BF16, rows, cols, m.bf16)
    return dev.upload(KF32, rows, cols, m.f32)


def stage_from_checkpoint(dev, ck: Checkpoint, ctx, rope_cos, rope_sin, first=0, last=None):
    """Layers [first, last) of a quantized checkpoint as an rkhip.Stage on
    dev (the reference moves a layer's matrices to the GPU and keeps its
    vectors beside them, model.go:345-387), plus the embedding and
    classifier uploaded for set_head. Returns (stage, matrices, embed,
    wcls); free the stage and every matrix before closing the device."""
    from . import Stage

    c = ck.config
    d, q, kv, h = c.dim, c.q_dim(), c.kv_dim(), c.hidden_dim
    shapes = {"wq": (q, d), "wk": (kv, d), "wv": (kv, d), "wo": (d, q), "w1": (h, d), "w2": (d, h), "w3": (h, d)}
    mats, layers = [], []
    for ly in ck.layers[first:last]:
        entry = {}
        for n, (rows, cols) in shapes.items():
            entry[n] = upload_matrix(dev, getattr(ly, n), rows, cols)
            mats.append(entry[n])
        for n in ("rms_att", "rms_ffn", "bq", "bk", "bv", "q_norm", "k_norm"):
            if getattr(ly, n) is not None:
                entry[n] = getattr(ly, n)
        layers.append(entry)
    st = Stage(dev, c.dim, c.hidden_dim, c.n_heads, c.n_kv_heads, ctx, layers, rope_cos, rope_sin,
               head_dim=c.head_dim, norm_eps=float(F32(c.norm_eps if c.norm_eps > 0 else 1e-5)),
               qkv_bias=c.qkv_bias, qk_norm=c.qk_norm)
    embed = upload_matrix(dev, ck.embed, c.vocab_size, c.dim)
    wcls = embed if c.shared_classifier else upload_matrix(dev, ck.head.wcls, c.vocab_size, c.dim)
    mats.append(embed)
    if wcls is not embed:
        mats.append(wcls)
    return st, mats, embed, wcls
