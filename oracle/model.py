"""Model-level CPU oracle: llama-family stages through rko_forward.

TEST INFRASTRUCTURE ONLY (see rk_oracle.h). Builds deterministic random
models, quantizes them as internal/llm/model.go:678-700 (Checkpoint.Quantize)
does, and runs tokens through the C restatement of Stage.Forward
(internal/llm/model.go:522-613), the head (:667-673) and Embed (:660-664).
"""
import ctypes
from dataclasses import dataclass

import numpy as np

from . import oracle

P = ctypes.c_void_p


class RkoMat(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("rows", ctypes.c_int32), ("cols", ctypes.c_int32), ("pad", ctypes.c_int32),
                ("f32", P), ("bf16", P), ("q8", P), ("q4", P), ("scales", P)]


class RkoLayer(ctypes.Structure):
    _fields_ = [(n, P) for n in ("rms_att", "rms_ffn", "bq", "bk", "bv", "q_norm", "k_norm")] + \
               [(n, RkoMat) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3")] + \
               [("experts", ctypes.c_int32), ("topk", ctypes.c_int32), ("router", RkoMat),
                ("ew1", P), ("ew2", P), ("ew3", P)]


class RkoConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("dim", "hidden", "layers", "heads", "kv_heads", "vocab", "seq_len",
                                              "head_dim")] + \
               [("rope_theta", ctypes.c_double), ("norm_eps", ctypes.c_double), ("qkv_bias", ctypes.c_int32),
                ("qk_norm", ctypes.c_int32)]


F32, BF16, Q8, Q4 = 0, 1, 2, 3


@dataclass
class Config:
    """internal/llm/model.go:37-64."""
    dim: int
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    vocab: int
    seq_len: int
    head_dim: int = 0
    rope_theta: float = 0.0
    norm_eps: float = 0.0
    qkv_bias: bool = False
    qk_norm: bool = False
    dtype: str = ""

    def head_size(self):
        return self.head_dim if self.head_dim > 0 else self.dim // self.heads

    def q_dim(self):
        return self.heads * self.head_size()

    def kv_dim(self):
        return self.kv_heads * self.head_size()

    def eps(self):
        return np.float32(self.norm_eps) if self.norm_eps > 0 else np.float32(1e-5)

    def embed_type(self):
        return "q8_0" if self.dtype in ("q4_0", "q4_m") else self.dtype

    def mat_type(self, sensitive):
        if self.dtype != "q4_m":
            return self.dtype
        return "q8_0" if sensitive else "q4_0"

    def ctype(self):
        return RkoConfig(self.dim, self.hidden, self.layers, self.heads, self.kv_heads, self.vocab, self.seq_len,
                         self.head_dim, self.rope_theta, self.norm_eps, int(self.qkv_bias), int(self.qk_norm))


class Mat:
    """A weight matrix in one storage type (internal/llm/model.go:133-148)."""

    def __init__(self, rows, cols, f32=None, dtype="f32"):
        self.rows, self.cols = rows, cols
        self.kind, self.f32, self.bf16, self.q, self.scales = F32, None, None, None, None
        if dtype in ("", "f32"):
            self.f32 = np.ascontiguousarray(f32, np.float32)
        elif dtype == "q8_0":
            self.kind = Q8
            self.q, self.scales = oracle.quantize8(f32)
        elif dtype == "q4_0":
            self.kind = Q4
            self.q, self.scales = oracle.quantize4(f32)
        elif dtype == "bf16":
            self.kind = BF16
            L = oracle.lib()
            self.bf16 = np.array([L.rko_to_bf16(np.float32(v)) for v in np.ravel(f32)], np.uint16)
        else:
            raise ValueError(dtype)

    @classmethod
    def from_codes(cls, kind, rows, cols, q, scales):
        m = cls.__new__(cls)
        m.rows, m.cols, m.kind, m.f32, m.bf16 = rows, cols, kind, None, None
        m.q, m.scales = q, scales
        return m

    def ctype(self):
        a = lambda x: x.ctypes.data if x is not None else None  # noqa: E731
        return RkoMat(self.kind, self.rows, self.cols, 0, a(self.f32), a(self.bf16),
                      a(self.q) if self.kind == Q8 else None, a(self.q) if self.kind == Q4 else None, a(self.scales))


class Moe:
    """A mixture-of-experts feed-forward (the build's contract, rko_moe_ffn):
    a router Mat [experts][dim] and per expert W1/W3 [hidden][dim] and W2
    [dim][hidden] Mats, top `topk`."""

    def __init__(self, router, w1, w2, w3, topk):
        self.router, self.w1, self.w2, self.w3, self.topk = router, list(w1), list(w2), list(w3), topk
        n = len(self.w1)
        arr = lambda ms: (RkoMat * n)(*[m.ctype() for m in ms])  # noqa: E731
        self._c = (arr(self.w1), arr(self.w2), arr(self.w3))  # kept alive with the layer


class Layer:
    VECS = ("rms_att", "rms_ffn", "bq", "bk", "bv", "q_norm", "k_norm")
    MATS = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")

    def __init__(self):
        for n in self.VECS + self.MATS:
            setattr(self, n, None)
        self.moe = None  # a Moe in place of w1/w2/w3

    def ctype(self):
        v = {n: (getattr(self, n).ctypes.data if getattr(self, n) is not None else None) for n in self.VECS}
        if self.moe is None:
            m = {n: getattr(self, n).ctype() for n in self.MATS}
            return RkoLayer(**v, **m)
        m = {n: (getattr(self, n).ctype() if getattr(self, n) is not None else RkoMat()) for n in self.MATS}
        a1, a2, a3 = self.moe._c
        return RkoLayer(**v, **m, experts=len(self.moe.w1), topk=self.moe.topk, router=self.moe.router.ctype(),
                        ew1=ctypes.addressof(a1), ew2=ctypes.addressof(a2), ew3=ctypes.addressof(a3))


def random_model(c: Config, seed: int, wscale=0.1):
    """A random model: matrices N(0, wscale), norm weights and biases N(0, 1),
    embedding N(0, 1), shared classifier (as model_test.go:250-270's
    randomModel, with numpy's generator). Returns float32 arrays."""
    rng = np.random.default_rng(seed)
    r = lambda n, s: (rng.normal(0, 1, n) * s).astype(np.float32)  # noqa: E731
    d, q, kv, h, hs = c.dim, c.q_dim(), c.kv_dim(), c.hidden, c.head_size()
    m = {"embed": r(c.vocab * d, 1.0), "rms_final": r(d, 1.0), "layers": []}
    for _ in range(c.layers):
        L = {"rms_att": r(d, 1.0), "wq": r(q * d, wscale), "wk": r(kv * d, wscale), "wv": r(kv * d, wscale),
             "wo": r(d * q, wscale), "rms_ffn": r(d, 1.0), "w1": r(h * d, wscale), "w2": r(d * h, wscale),
             "w3": r(h * d, wscale)}
        if c.qkv_bias:
            L.update(bq=r(q, 1.0), bk=r(kv, 1.0), bv=r(kv, 1.0))
        if c.qk_norm:
            L.update(q_norm=r(hs, 1.0), k_norm=r(hs, 1.0))
        m["layers"].append(L)
    return m


class Model:
    """A model in its storage types (Checkpoint after Quantize)."""

    def __init__(self, c: Config, raw):
        self.c = c
        d, q, kv, h = c.dim, c.q_dim(), c.kv_dim(), c.hidden
        self.embed = Mat(c.vocab, d, raw["embed"], c.embed_type())
        # a separate classifier when raw has one, else the shared embedding
        self.wcls = Mat(c.vocab, d, raw["wcls"], c.embed_type()) if raw.get("wcls") is not None else self.embed
        self.rms_final = raw["rms_final"]
        self.layers = []
        shapes = {"wq": (q, d, False), "wk": (kv, d, False), "wv": (kv, d, True), "wo": (d, q, False),
                  "w1": (h, d, False), "w2": (d, h, True), "w3": (h, d, False)}
        for L in raw["layers"]:
            ly = Layer()
            for n in Layer.VECS:
                if n in L:
                    setattr(ly, n, L[n])
            for n, (rows, cols, sens) in shapes.items():
                setattr(ly, n, Mat(rows, cols, L[n], c.mat_type(sens)))
            self.layers.append(ly)

    def rope(self, n):
        half = self.c.head_size() // 2
        cos = np.empty(n * half, np.float32)
        sin = np.empty(n * half, np.float32)
        cc = self.c.ctype()
        oracle.lib().rko_rope_table(ctypes.byref(cc), n, oracle.ptr(cos), oracle.ptr(sin))
        return cos, sin

    def embed_token(self, tok):
        x = np.empty(self.c.dim, np.float32)
        cc, mt = self.c.ctype(), self.embed.ctype()
        oracle.lib().rko_embed(ctypes.byref(cc), ctypes.byref(mt), tok, oracle.ptr(x))
        return x

    def logits(self, x):
        out = np.empty(self.c.vocab, np.float32)
        cc, mt = self.c.ctype(), self.wcls.ctype()
        x = np.ascontiguousarray(x, np.float32)
        oracle.lib().rko_logits(ctypes.byref(cc), oracle.ptr(self.rms_final), ctypes.byref(mt), oracle.ptr(x),
                                oracle.ptr(out))
        return out


class Stage:
    """Layers [first, last) with their key/value caches (internal/llm Stage)."""

    def __init__(self, model: Model, ctx, first=0, last=None):
        c = model.c
        self.m, self.c, self.ctx = model, c, ctx
        self.layers = model.layers[first:last]
        self.cos, self.sin = model.rope(ctx)
        self._cl = (RkoLayer * len(self.layers))(*[ly.ctype() for ly in self.layers])
        self.keys = [np.zeros(ctx * c.kv_dim(), np.float32) for _ in self.layers]
        self.vals = [np.zeros(ctx * c.kv_dim(), np.float32) for _ in self.layers]
        self._kp = (P * len(self.layers))(*[k.ctypes.data for k in self.keys])
        self._vp = (P * len(self.layers))(*[v.ctypes.data for v in self.vals])
        self._cc = c.ctype()
        n = 3 * c.dim + 2 * c.q_dim() + 2 * c.kv_dim() + 2 * c.hidden + ctx
        self._scratch = np.zeros(n, np.float32)

    def forward(self, x, pos):
        """One token at pos, x in place (and returned)."""
        x = np.ascontiguousarray(x, np.float32)
        oracle.lib().rko_forward(ctypes.byref(self._cc), self._cl, len(self.layers), oracle.ptr(self.cos),
                                 oracle.ptr(self.sin), self._kp, self._vp, self.ctx, oracle.ptr(x), pos,
                                 oracle.ptr(self._scratch))
        return x
