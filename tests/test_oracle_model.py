"""Pins the oracle's layer forward (internal/llm/model.go:522-673) on the CPU:
an independent float64 forward of the architecture (the reference's
TestForwardMatchesNaiveReference, model_test.go:50-171), stage-split
invariance (TestStagesComposeExactly, :175-195), and the deviation of
quantized models from the float model (TestQuantizedModels, :197-248)."""
import math

import numpy as np

from oracle.model import Config, Model, Stage, random_model


def naive_logits(c: Config, raw, tokens):
    """float64 forward over a whole sequence, from the architecture's
    definition (RMSNorm, RoPE on adjacent pairs, GQA attention, SwiGLU),
    not from the engine."""
    hs = c.head_size()
    theta = c.rope_theta if c.rope_theta > 0 else 10000.0
    eps = c.norm_eps if c.norm_eps > 0 else 1e-5
    f = lambda v: np.asarray(v, np.float64)  # noqa: E731

    def mv(w, x, rows):
        return f(w).reshape(rows, -1) @ x

    def norm(x, w):
        return f(w) * x / math.sqrt(np.mean(x * x) + eps)

    def rope(v, pos):
        v = v.copy()
        for i in range(0, len(v), 2):
            th = pos * theta ** (-(i % hs) / hs)
            a, b = v[i], v[i + 1]
            v[i], v[i + 1] = a * math.cos(th) - b * math.sin(th), a * math.sin(th) + b * math.cos(th)
        return v

    caches = [([], []) for _ in range(c.layers)]
    x = None
    for pos, tok in enumerate(tokens):
        x = f(raw["embed"][tok * c.dim:(tok + 1) * c.dim])
        for li, L in enumerate(raw["layers"]):
            xn = norm(x, L["rms_att"])
            q, k, v = mv(L["wq"], xn, c.q_dim()), mv(L["wk"], xn, c.kv_dim()), mv(L["wv"], xn, c.kv_dim())
            if c.qkv_bias:
                q, k, v = q + f(L["bq"]), k + f(L["bk"]), v + f(L["bv"])
            if c.qk_norm:
                q = np.concatenate([norm(q[h:h + hs], L["q_norm"]) for h in range(0, len(q), hs)])
                k = np.concatenate([norm(k[h:h + hs], L["k_norm"]) for h in range(0, len(k), hs)])
            q, k = rope(q, pos), rope(k, pos)
            caches[li][0].append(k)
            caches[li][1].append(v)
            att = np.zeros(c.q_dim())
            for h in range(c.heads):
                g = h // (c.heads // c.kv_heads)
                sc = np.array([q[h * hs:(h + 1) * hs] @ kk[g * hs:(g + 1) * hs] for kk in caches[li][0]]) / math.sqrt(hs)
                p = np.exp(sc - sc.max())
                p /= p.sum()
                for t, vv in enumerate(caches[li][1]):
                    att[h * hs:(h + 1) * hs] += p[t] * vv[g * hs:(g + 1) * hs]
            x = x + mv(L["wo"], att, c.dim)
            xn = norm(x, L["rms_ffn"])
            a, b = mv(L["w1"], xn, c.hidden), mv(L["w3"], xn, c.hidden)
            x = x + mv(L["w2"], a / (1 + np.exp(-a)) * b, c.dim)
    return mv(raw["embed"], norm(x, raw["rms_final"]), c.vocab)


CONFIGS = [
    Config(dim=32, hidden=72, layers=3, heads=4, kv_heads=2, vocab=50, seq_len=24),
    Config(dim=64, hidden=128, layers=2, heads=4, kv_heads=2, vocab=50, seq_len=24, qkv_bias=True),
    Config(dim=64, hidden=96, layers=2, heads=4, kv_heads=2, vocab=50, seq_len=24, head_dim=32, qk_norm=True,
           rope_theta=1e6, norm_eps=1e-6),
]


def test_forward_matches_naive_float64_reference():
    tokens = [1, 7, 33, 2, 49, 12, 12, 30, 5, 18]
    for c in CONFIGS:
        raw = random_model(c, 1, wscale=0.2)
        m = Model(c, raw)
        st = Stage(m, c.seq_len)
        for pos, tok in enumerate(tokens):
            x = st.forward(m.embed_token(tok), pos)
            got = m.logits(x)
            want = naive_logits(c, raw, tokens[:pos + 1])
            assert np.max(np.abs(got - want)) <= 1e-3, (c, pos)
            assert int(np.argmax(got)) == int(np.argmax(want))


def test_stages_compose_exactly():
    for c in CONFIGS:
        for dtype in ("", "q8_0", "q4_m"):
            c2 = Config(**{**c.__dict__, "dtype": dtype})
            m = Model(c2, random_model(c2, 2))
            whole = Stage(m, c2.seq_len)
            split = [Stage(m, c2.seq_len, 0, 1), Stage(m, c2.seq_len, 1, None)]
            for pos, tok in enumerate([1, 4, 9, 16, 25]):
                a = whole.forward(m.embed_token(tok), pos)
                b = m.embed_token(tok)
                for s in split:
                    b = s.forward(b, pos)
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_quantized_models_stay_close_to_float():
    c = Config(dim=64, hidden=128, layers=3, heads=4, kv_heads=2, vocab=50, seq_len=24)
    raw = random_model(c, 7)
    exact = Model(c, raw)
    es = Stage(exact, 8)
    worst = {}
    for dtype in ("q8_0", "q4_m", "q4_0"):
        cq = Config(**{**c.__dict__, "dtype": dtype})
        mq = Model(cq, raw)
        qs = Stage(mq, 8)
        es = Stage(exact, 8)
        w = 0.0
        for pos, tok in enumerate([1, 4, 9, 16, 25]):
            a = qs.forward(mq.embed_token(tok), pos)
            e = es.forward(exact.embed_token(tok), pos)
            w = max(w, float(np.max(np.abs(a - e) / (1 + np.abs(e)))))
        worst[dtype] = w
        assert w <= 0.5, (dtype, w)
    assert worst["q8_0"] < worst["q4_0"]
