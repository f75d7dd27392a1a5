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


# --- closed forms for the order of the layer's float sums -------------------
# Each input makes the reference's order give one float32 and every other
# plausible order (pairwise, reversed, a plain dot product) another.

def _b(v):
    return np.asarray(v, np.float32).view(np.uint32)


def test_softmax_sums_in_one_sequential_chain():
    """internal/llm/model.go:640-654: sum += e_i for i ascending. With
    e = 1, Exp32(-17), Exp32(-17), each small term is below half an ulp of 1
    (2^-24), so 1 + e1 + e2 stays 1 and p0 = 1 exactly; added as
    1 + (e1 + e2) or from the end, the two terms pass half an ulp and the
    sum is 1 + 2^-23, so p0 = Recip32(1 + 2^-23) < 1."""
    from oracle import oracle

    e = np.float32(oracle.exp32(-17.0))
    assert 2.0 ** -25 < e <= 2.0 ** -24
    assert np.float32(np.float32(1) + np.float32(e + e)) == np.float32(1 + 2.0 ** -23)
    for x in ([0.0, -17.0, -17.0], [5.0, -12.0, -12.0]):  # the maximum subtracted first
        p = oracle.softmax(np.array(x, np.float32))
        assert _b(p[0]) == _b(1.0), p
        assert _b(p[1]) == _b(e) and _b(p[2]) == _b(e)


def test_attention_adds_positions_in_order():
    """internal/llm/model.go:580-586: out[i] += a_t·v_t[i] for t ascending,
    from +0. A zero query gives equal scores, weights Recip32(4) = 0.25
    exactly, and exact products. Element 0's products 1e8, 1, -1e8, 1 sum
    to 1 in order ((1e8 + 1) rounds to 1e8) but to 0 reversed or pairwise;
    element 1's 1, 1e8, -1e8, 0 sum to 0 in order but to 1 reversed."""
    from oracle import oracle

    hs = 32
    keys = np.random.default_rng(1).normal(0, 1, (4, hs)).astype(np.float32)
    vals = np.zeros((4, hs), np.float32)
    vals[:, 0] = np.array([1e8, 1, -1e8, 1], np.float32) * 4
    vals[:, 1] = np.array([1, 1e8, -1e8, 0], np.float32) * 4
    vals[:, 2] = 4.0
    att, out = oracle.attention_head(np.zeros(hs, np.float32), keys, vals, 1 / math.sqrt(hs))
    assert np.all(_b(att) == _b(0.25))
    assert _b(out[0]) == _b(1.0) and _b(out[1]) == _b(0.0) and _b(out[2]) == _b(4.0)
    assert not out[3:].any()


def test_rmsnorm_uses_dot32():
    """internal/llm/model.go:632-638: ss = Dot32(x, x)·Recip32(n) + eps.
    x = 4096 then 31 ones: Dot32's running sum 0 holds 2^24, its combine
    adds the ones in groups (e_0 = (2^24 + 1) + (1 + 1) = 2^24 + 2, the other
    seven 4 each), giving 2^24 + 30; a sequential Dot loses every one
    (2^24 + 1 is a tie that rounds back to 2^24). The output is
    w·float32(Rsqrt32(ss)·x) from the Dot32 sum, not from the other."""
    from oracle import oracle

    x = np.ones(32, np.float32)
    x[0] = 4096
    assert oracle.dot32(x, x) == np.float32(2 ** 24 + 30)
    assert np.float32(oracle.lib().rko_dot(oracle.ptr(x), oracle.ptr(x), 32)) == np.float32(2 ** 24)
    w = np.linspace(0.5, 1.5, 32).astype(np.float32)
    eps = np.float32(1e-5)
    rn = np.float32(oracle.recip32(32.0))
    assert rn == np.float32(1 / 32)

    def norm_from(total):
        ss = np.float32(np.float32(np.float32(total) * rn) + eps)
        r = np.float32(oracle.rsqrt32(ss))
        return (w * (r * x).astype(np.float32)).astype(np.float32)

    got = oracle.rmsnorm(x, w, eps)
    assert np.array_equal(_b(got), _b(norm_from(2 ** 24 + 30)))
    assert not np.array_equal(_b(got), _b(norm_from(2 ** 24)))


def test_forward_with_threaded_products_gives_the_same_bits():
    """The forward's products through the AVX2 block sums on several
    threads (used by the model-size GPU checks) give the portable loops'
    bits, for Q8 and Q4 layers."""
    import pytest
    from oracle import oracle

    if not oracle.lib().rko_have_avx2():
        pytest.skip("no AVX2 on this host")
    for dtype in ("q8_0", "q4_m"):
        c = Config(**{**CONFIGS[0].__dict__, "dtype": dtype})
        m = Model(c, random_model(c, 11))
        outs = []
        for threads in (0, 5):
            st = Stage(m, 24)
            with oracle.matvec_threads(threads):
                xs = [m.logits(st.forward(m.embed_token(t), pos)) for pos, t in enumerate([3, 7, 1, 40, 2])]
            outs.append(np.stack(xs).view(np.uint32))
        assert np.array_equal(outs[0], outs[1])
