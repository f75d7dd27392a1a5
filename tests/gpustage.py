"""The reference's GPU stage (internal/llm/gpustage.go) driven through the
Batch C-ABI, operation for operation: what internal/llm keeps doing on top
of the cgo shim. Used by the stage parity tests."""

import numpy as np

import rkhip
from oracle import oracle

GPU_BATCH = 64  # gpustage.go:17


class GPUStage:
    def __init__(self, dev, model, ctx, first=0, last=None):
        c = model.c
        self.dev, self.c, self.ctx = dev, c, ctx
        self.layers = model.layers[first:last]
        self.mats, self.vecs, self.offs = [], [], None
        for ly in self.layers:
            up = {}
            for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"):
                m = getattr(ly, n)
                w = {rkhip.F32: m.f32, rkhip.BF16: m.bf16}.get(m.kind, m.q)  # the Matrix's storage (model.go:133-148)
                up[n] = dev.upload(m.kind, m.rows, m.cols, w, m.scales)
            self.mats.append(up)
            # gpustage.go vecLayout (model.go:297-313)
            allv, offs, at = [], {}, 0
            for n in ("rms_att", "rms_ffn") + (("bq", "bk", "bv") if c.qkv_bias else ()) + \
                     (("q_norm", "k_norm") if c.qk_norm else ()):
                offs[n] = at
                allv.append(getattr(ly, n))
                at += getattr(ly, n).size
            self.offs = offs
            self.vecs.append(dev.upload_vectors(np.concatenate(allv)))
        # gpustage.go:51-83 arena layout
        at = 0

        def alloc(n):
            nonlocal at
            o = at
            at += n
            return o

        self.x, self.xb, self.xb2 = alloc(c.dim), alloc(c.dim), alloc(c.dim)
        self.q, self.k, self.v, self.att_out = alloc(c.q_dim()), alloc(c.kv_dim()), alloc(c.kv_dim()), alloc(c.q_dim())
        self.hb, self.hb2 = alloc(c.hidden), alloc(c.hidden)
        self.att = alloc(c.heads * ctx)
        widest = max(c.dim, c.q_dim(), c.hidden)
        qx, xs = alloc(widest // 4), alloc(widest // 32)
        half = c.head_size() // 2
        self.cos, self.sin = alloc(ctx * half), alloc(ctx * half)
        self.keys = [alloc(ctx * c.kv_dim()) for _ in self.layers]
        self.vals = [alloc(ctx * c.kv_dim()) for _ in self.layers]
        staging = max(2 * GPU_BATCH * c.dim, 2 * ctx * half)
        self.arena = dev.arena(at, staging)
        self.arena.set_quant_scratch(qx, xs)
        cos, sin = model.rope(ctx)
        b = self.arena.begin()
        b.write(self.cos, cos[:ctx * half])
        b.write(self.sin, sin[:ctx * half])
        b.submit()

    def close(self):
        self.arena.free()
        for v in self.vecs:
            v.free()
        for up in self.mats:
            for m in up.values():
                m.free()

    def forward(self, xs, pos, tokens):
        """gpustage.go:100-116: xs (tokens x dim) in place, 64 a submission."""
        c = self.c
        xs = np.ascontiguousarray(xs, np.float32).reshape(tokens, c.dim)
        for start in range(0, tokens, GPU_BATCH):
            n = min(GPU_BATCH, tokens - start)
            b = self.arena.begin()
            outs = []
            for t in range(n):
                b.write(self.x, xs[start + t])
                self.token(b, pos + start + t)
                outs.append(b.read(self.x, c.dim))
            b.submit()
            for t in range(n):
                xs[start + t] = outs[t]
        return xs

    def token(self, b, pos):
        """gpustage.go:119-152."""
        c = self.c
        hs, q_dim, kv_dim = c.head_size(), c.q_dim(), c.kv_dim()
        eps = c.eps()
        recip_dim = oracle.recip32(np.float32(c.dim))  # num.Recip32, computed by the Go host
        recip_head = oracle.recip32(np.float32(hs))
        inv_sqrt = rkhip.inv_sqrt_head(hs)
        half = hs // 2
        o = self.offs
        for li in range(len(self.layers)):
            m, vec = self.mats[li], self.vecs[li]
            b.rmsnorm(vec, self.x, self.xb, o["rms_att"], c.dim, 1, 0, recip_dim, eps)
            b.matvecs([m["wq"], m["wk"], m["wv"]], [self.q, self.k, self.v], self.xb)
            if c.qkv_bias:
                b.addvec(vec, self.q, o["bq"], q_dim)
                b.addvec(vec, self.k, o["bk"], kv_dim)
                b.addvec(vec, self.v, o["bv"], kv_dim)
            if c.qk_norm:
                b.rmsnorm(vec, self.q, self.q, o["q_norm"], hs, c.heads, hs, recip_head, eps)
                b.rmsnorm(vec, self.k, self.k, o["k_norm"], hs, c.kv_heads, hs, recip_head, eps)
            b.rope(self.q, self.k, q_dim, kv_dim, hs, self.cos + pos * half, self.sin + pos * half)
            b.copy(self.k, self.keys[li] + pos * kv_dim, kv_dim)
            b.copy(self.v, self.vals[li] + pos * kv_dim, kv_dim)
            b.attention(self.q, self.keys[li], self.vals[li], self.att, self.ctx, self.att_out, pos + 1, c.heads,
                        c.kv_heads, hs, kv_dim, inv_sqrt)
            b.matvecs([m["wo"]], [self.xb2], self.att_out)
            b.residual(self.x, self.xb2, c.dim, False)
            b.rmsnorm(vec, self.x, self.xb, o["rms_ffn"], c.dim, 1, 0, recip_dim, eps)
            b.matvecs([m["w1"], m["w3"]], [self.hb, self.hb2], self.xb)
            b.silumul(self.hb, self.hb2, c.hidden)
            b.matvecs([m["w2"]], [self.xb], self.hb)
            b.residual(self.x, self.xb, c.dim, True)
