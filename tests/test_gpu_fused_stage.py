"""The fused stage (rk_stage_*) gives the CPU oracle's bits.

* The device's restatements of package num's float functions, over inputs
  that reach every branch (specials, denormals, both overflow bounds).
* Stage.ForwardMany through the fused launches and graph replays, for the
  three architecture variants of the reference's TestGPUStagesMatchCPU
  (internal/llm/gpu_test.go:32-111) in each weight type.
* Greedy generation entirely on the device (embedding, layers, head,
  argmax, position advance) against the oracle's token loop, every logit of
  every step compared bitwise: config 1 (llama2.c 288, 128 tokens after 8
  prompt ids), and one layer at the 8B, Qwen-7B (Q4) and Qwen3 (QK-norm,
  q_dim != dim) attention/FFN shapes with their full vocabularies.
"""
import numpy as np
import pytest

import rkhip
from oracle import oracle
from oracle.model import Config, Layer, Mat, Model, Stage, random_model, Q8, Q4

pytestmark = pytest.mark.gpu

CONFIGS = [
    Config(dim=64, hidden=128, layers=3, heads=4, kv_heads=2, vocab=50, seq_len=96, qkv_bias=True),
    Config(dim=64, hidden=96, layers=2, heads=4, kv_heads=2, vocab=50, seq_len=96, head_dim=32, qk_norm=True,
           rope_theta=1e6, norm_eps=1e-6),
    Config(dim=96, hidden=160, layers=2, heads=3, kv_heads=3, vocab=50, seq_len=96),
]


def same_bits(a, b, what):
    a = np.ascontiguousarray(a, np.float32).view(np.uint32)
    b = np.ascontiguousarray(b, np.float32).view(np.uint32)
    if not np.array_equal(a, b):
        i = int(np.argmax(a != b))
        raise AssertionError(f"{what}: first difference at {i}: {a.view(np.float32)[i]!r} vs "
                             f"{b.view(np.float32)[i]!r} ({int(np.sum(a != b))} differ)")


def num_inputs(rng, lo_exp, hi_exp):
    """Random magnitudes over [2^lo, 2^hi] of both signs, plus specials and
    denormals."""
    mag = np.exp2(rng.uniform(lo_exp, hi_exp, 400000)).astype(np.float32)
    sgn = np.where(rng.random(mag.size) < 0.5, -1, 1).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, 4.0, 2.0, 0.5, 1e-45, -1e-45, 1.1754942e-38,
                        3.4028235e38, -3.4028235e38], np.float32)
    den = (rng.integers(1, 1 << 23, 2000, dtype=np.int64)).astype(np.uint32).view(np.float32)
    return np.concatenate([mag * sgn, special, den, -den])


@pytest.mark.parametrize("fn,lo,hi", [(rkhip.FN_RECIP32, -149, 127), (rkhip.FN_RSQRT32, -149, 127),
                                      (rkhip.FN_EXP32, -12, 7), (rkhip.FN_SILU, -12, 7)])
def test_num_functions_match_oracle(dev, fn, lo, hi):
    x = num_inputs(np.random.default_rng(fn + 40), lo, hi)
    if fn in (rkhip.FN_EXP32, rkhip.FN_SILU):  # both bounds of Exp32 (88.72, -103.97) and around them
        x = np.concatenate([x, np.linspace(-110, 95, 20001, dtype=np.float32)])
    same_bits(dev.num_eval(fn, x), oracle.num_eval(fn, x), f"fn {fn}")


def upload_layers(dev, m):
    layers, mats = [], []
    for ly in m.layers:
        d = {}
        for n in Layer.MATS:
            mt = getattr(ly, n)
            d[n] = dev.upload(mt.kind, mt.rows, mt.cols, mt.q, mt.scales)
            mats.append(d[n])
        for n in Layer.VECS:
            d[n] = getattr(ly, n)
        layers.append(d)
    return layers, mats


def make_stage(dev, m, ctx):
    c = m.c
    layers, mats = upload_layers(dev, m)
    cos, sin = m.rope(ctx)
    st = rkhip.Stage(dev, c.dim, c.hidden, c.heads, c.kv_heads, ctx, layers, cos, sin, head_dim=c.head_dim,
                     norm_eps=float(c.eps()), qkv_bias=c.qkv_bias, qk_norm=c.qk_norm)
    return st, mats


@pytest.mark.parametrize("ci", range(len(CONFIGS)))
@pytest.mark.parametrize("dtype", ["q8_0", "q4_m", "q4_0"])
def test_fused_stage_forward_matches_cpu(dev, ci, dtype):
    c = Config(**{**CONFIGS[ci].__dict__, "dtype": dtype})
    m = Model(c, random_model(c, 9))
    cpu = Stage(m, 80)
    gpu, mats = make_stage(dev, m, 80)
    prompt = [(i * 7 + 3) % c.vocab for i in range(70)]
    a = np.stack([m.embed_token(t) for t in prompt])
    b = gpu.forward(a, 0)
    for pos in range(len(prompt)):
        a[pos] = cpu.forward(a[pos], pos)
        same_bits(b[pos], a[pos], f"prompt position {pos}")
    for i, tok in enumerate([16, 25, 36, 49, 7, 3]):
        pos = len(prompt) + i
        x = cpu.forward(m.embed_token(tok), pos)
        y = gpu.forward(m.embed_token(tok), pos)[0]
        same_bits(y, x, f"decode position {pos}")
    gpu.free()
    for mt in mats:
        mt.free()
    assert dev.used == 0


def oracle_generate(m, prompt, steps, ctx):
    """The coordinator's greedy loop on the CPU: Embed, Stage.Forward, Head.Logits, argmax."""
    st = Stage(m, ctx)
    toks, logits = list(prompt), []
    for pos in range(len(prompt) + steps - 1):
        x = st.forward(m.embed_token(toks[pos]), pos)
        if pos + 1 >= len(prompt):
            lg = m.logits(x)
            logits.append(lg)
            toks.append(oracle.argmax(lg))
    return toks[len(prompt):], logits


def gpu_generate(dev, m, prompt, steps, ctx):
    gpu, mats = make_stage(dev, m, ctx)
    emb = dev.upload(m.embed.kind, m.embed.rows, m.embed.cols, m.embed.q, m.embed.scales)
    gpu.set_head(emb, emb, m.rms_final)
    gpu.generate_start(prompt)
    if len(prompt) > 1:
        gpu.generate_run(len(prompt) - 1)
    logits = [gpu.generate_run(1, want_logits=True)[0] for _ in range(steps)]
    toks = gpu.tokens(len(prompt), steps)
    # the same generation again, replayed without stops: the same tokens
    again = gpu.generate(prompt, steps)
    gpu.free()
    emb.free()
    for mt in mats:
        mt.free()
    return list(toks), logits, list(again)


def check_generation(dev, m, prompt, steps, ctx):
    want_t, want_l = oracle_generate(m, prompt, steps, ctx)
    got_t, got_l, again = gpu_generate(dev, m, prompt, steps, ctx)
    for k in range(steps):
        same_bits(got_l[k], want_l[k], f"logits of step {k}")
    assert got_t == want_t
    assert again == want_t
    assert dev.used == 0


def llama2c_model(seed=1):
    """Config 1: llama2.c 288/6/6/768, vocab 32000; f32 weights N(0, 0.02)
    from the seed, norm weights 1, quantized to q8_0 (Checkpoint.Quantize)."""
    c = Config(dim=288, hidden=768, layers=6, heads=6, kv_heads=6, vocab=32000, seq_len=256, dtype="q8_0")
    rng = np.random.default_rng(seed)
    r = lambda n: (rng.normal(0, 0.02, n)).astype(np.float32)  # noqa: E731
    d, h = c.dim, c.hidden
    raw = {"embed": r(c.vocab * d), "rms_final": np.ones(d, np.float32), "layers": []}
    for _ in range(c.layers):
        raw["layers"].append({"rms_att": np.ones(d, np.float32), "wq": r(d * d), "wk": r(d * d), "wv": r(d * d),
                              "wo": r(d * d), "rms_ffn": np.ones(d, np.float32), "w1": r(h * d), "w2": r(d * h),
                              "w3": r(h * d)})
    return Model(c, raw)


def test_generation_config1_128_tokens(dev):
    m = llama2c_model(1)
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, 32000, 8)]
    check_generation(dev, m, prompt, 128, 256)


def test_generation_q4m_qwen2_and_qwen3_variants(dev):
    for ci in (0, 1):
        c = Config(**{**CONFIGS[ci].__dict__, "dtype": "q4_m"})
        m = Model(c, random_model(c, 3))
        check_generation(dev, m, [1, 5, 9, 2], 40, 96)


def coded_model(c, seed, scale_lo=1e-4, scale_hi=1e-3):
    """Random codes and scales directly (as config 2's matrices): Q8 (or
    Q4 for q4_0 layers), norm weights N(1, 0.1), embedding/classifier Q8."""
    rng = np.random.default_rng(seed)
    m = Model.__new__(Model)
    m.c = c

    def mat(rows, cols, kind):
        s = rng.uniform(scale_lo, scale_hi, rows * cols // 32).astype(np.float32)
        # uniform random bytes, from the generator's raw 64-bit words (fast
        # at model sizes); Q8 codes are never -128 (quantize8 clamps to ±127)
        n = rows * cols if kind == Q8 else rows * cols // 2
        q = rng.bit_generator.random_raw((n + 7) // 8).view(np.uint8)[:n].copy()
        if kind == Q8:
            q = q.view(np.int8)
            q[q == -128] = -127
        return Mat.from_codes(kind, rows, cols, q, s)

    kind = Q4 if c.dtype == "q4_0" else Q8
    d, q, kv, h, hs = c.dim, c.q_dim(), c.kv_dim(), c.hidden, c.head_size()
    m.embed = mat(c.vocab, d, Q8)
    m.wcls = m.embed
    m.rms_final = rng.normal(1, 0.1, d).astype(np.float32)
    m.layers = []
    for _ in range(c.layers):
        ly = Layer()
        ly.rms_att = rng.normal(1, 0.1, d).astype(np.float32)
        ly.rms_ffn = rng.normal(1, 0.1, d).astype(np.float32)
        if c.qkv_bias:
            ly.bq, ly.bk, ly.bv = (rng.normal(0, 0.5, n).astype(np.float32) for n in (q, kv, kv))
        if c.qk_norm:
            ly.q_norm, ly.k_norm = (rng.normal(1, 0.1, hs).astype(np.float32) for _ in range(2))
        for n, (rows, cols) in {"wq": (q, d), "wk": (kv, d), "wv": (kv, d), "wo": (d, q), "w1": (h, d),
                                "w2": (d, h), "w3": (h, d)}.items():
            setattr(ly, n, mat(rows, cols, kind))
        m.layers.append(ly)
    return m


@pytest.mark.parametrize("name", ["llama8b", "qwen7b_q4", "qwen3_attn"])
def test_generation_real_shapes_one_layer(dev, name):
    if name == "llama8b":  # config 3's layer and head
        c = Config(dim=4096, hidden=14336, layers=1, heads=32, kv_heads=8, vocab=128256, seq_len=64,
                   rope_theta=500000.0, dtype="q8_0")
    elif name == "qwen7b_q4":  # config 4's layer (hidden 18944: the separate-quantize path) and head
        c = Config(dim=3584, hidden=18944, layers=1, heads=28, kv_heads=4, vocab=152064, seq_len=64,
                   rope_theta=1000000.0, qkv_bias=True, norm_eps=1e-6, dtype="q4_0")
    else:  # config 5's attention: q_dim 4096 != dim 2048, QK-norm; a dense FFN of the expert width
        c = Config(dim=2048, hidden=768, layers=1, heads=32, kv_heads=4, vocab=151936, seq_len=64, head_dim=128,
                   rope_theta=1000000.0, qk_norm=True, norm_eps=1e-6, dtype="q8_0")
    m = coded_model(c, 5)
    check_generation(dev, m, [11, 7000, 123, 99], 12, 64)


def test_generation_qk_norm_scores_in_the_values_launch_to_256(dev):
    """A QK-norm layer's decode step with head size 128 at contexts up to 256
    forms its scores inside the values-and-Wo launch (one quad of lanes a
    cached key, in rounds of 64 positions; one workgroup per kv head storing
    the position's k and v). Positions 99..255 reach every round, every logit
    bitwise."""
    c = Config(dim=256, hidden=128, layers=2, heads=32, kv_heads=4, vocab=64, seq_len=256, head_dim=128,
               rope_theta=1000000.0, qk_norm=True, norm_eps=1e-6, dtype="q8_0")
    m = coded_model(c, 12)
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, c.vocab, 100)]
    check_generation(dev, m, prompt, 156, 256)


@pytest.mark.parametrize("case", ["kv2_ctx1024", "kv2_ctx1100", "kv8_gqa_ctx1000"])
def test_generation_long_context(dev, case):
    """Decode at positions up to the end of a long context, every logit
    bitwise: contexts up to 1024 keep all of a value slice's positions in
    LDS (several product chunks), 1100 takes the chunked values kernel;
    8 value heads of 32 (two query heads each) put each value slice's
    workgroups on one XCD."""
    if case.startswith("kv2"):
        ctx = int(case.split("ctx")[1])
        c = Config(**{**CONFIGS[1].__dict__, "dtype": "q8_0", "seq_len": ctx})
    else:
        ctx = 1000
        c = Config(dim=128, hidden=192, layers=2, heads=16, kv_heads=8, vocab=50, seq_len=ctx, head_dim=32,
                   dtype="q8_0")
    m = Model(c, random_model(c, 6))
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, c.vocab, ctx - 10)]
    check_generation(dev, m, prompt, 10, ctx)


def test_generation_head128_to_context_end(dev):
    """Head size 128 (the 8B, Qwen and Qwen3 heads) decoding at positions up
    to the last of a 1024-position context: the largest context whose value
    slices stay in registers (four product chunks) and eight score tiles,
    every logit bitwise."""
    c = Config(dim=256, hidden=384, layers=2, heads=4, kv_heads=2, vocab=64, seq_len=1024, head_dim=128,
               dtype="q8_0")
    m = Model(c, random_model(c, 7))
    prompt = [int(t) for t in np.random.default_rng(4).integers(0, c.vocab, 1014)]
    check_generation(dev, m, prompt, 10, 1024)


def forward_one_by_one(st, xs, pos0):
    return np.stack([st.forward(xs[t], pos0 + t)[0] for t in range(len(xs))])


@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_batched_forward_matches_token_by_token(dev, ci):
    """A forward of many tokens (the batched prefill path: MFMA products,
    per-token norms and attention) equals one token at a time (the decode
    path), at a nonzero start position and over more tokens than one batch
    holds (256)."""
    c = Config(**{**CONFIGS[ci].__dict__, "dtype": "q4_m"})
    m = Model(c, random_model(c, 4))
    ctx = 600
    a, mats_a = make_stage(dev, m, ctx)
    b, mats_b = make_stage(dev, m, ctx)
    xs = np.stack([m.embed_token((i * 11 + 5) % c.vocab) for i in range(300)])
    head = forward_one_by_one(a, xs[:20], 0)
    same_bits(forward_one_by_one(b, xs[:20], 0), head, "first 20 positions")
    got = a.forward(xs[20:], 20)
    want = forward_one_by_one(b, xs[20:], 20)
    for t in range(len(want)):
        same_bits(got[t], want[t], f"position {20 + t}")
    # and decode continues from the batch's cache entries
    x = m.embed_token(3)
    same_bits(a.forward(x, 300)[0], b.forward(x, 300)[0], "decode after the batch")
    for st in (a, b):
        st.free()
    for mt in mats_a + mats_b:
        mt.free()
    assert dev.used == 0


@pytest.mark.parametrize("name", ["llama8b", "qwen7b_q4", "qwen3_attn"])
def test_batched_forward_real_shapes_one_layer(dev, name):
    """The prefill path at the 8B / Qwen-7B (Q4, QKV bias, hidden 18944) /
    Qwen3 (QK-norm, q_dim != dim) layer shapes: 130 tokens at once equal the
    decode path token by token, which the generation tests pin to the
    oracle."""
    if name == "llama8b":
        c = Config(dim=4096, hidden=14336, layers=1, heads=32, kv_heads=8, vocab=16, seq_len=160,
                   rope_theta=500000.0, dtype="q8_0")
    elif name == "qwen7b_q4":
        c = Config(dim=3584, hidden=18944, layers=1, heads=28, kv_heads=4, vocab=16, seq_len=160,
                   rope_theta=1000000.0, qkv_bias=True, norm_eps=1e-6, dtype="q4_0")
    else:
        c = Config(dim=2048, hidden=768, layers=1, heads=32, kv_heads=4, vocab=16, seq_len=160, head_dim=128,
                   rope_theta=1000000.0, qk_norm=True, norm_eps=1e-6, dtype="q8_0")
    m = coded_model(c, 6)
    rng = np.random.default_rng(2)
    xs = rng.normal(0, 1, (130, c.dim)).astype(np.float32)
    a, mats_a = make_stage(dev, m, 160)
    b, mats_b = make_stage(dev, m, 160)
    got = a.forward(xs, 0)
    want = forward_one_by_one(b, xs, 0)
    for t in range(len(want)):
        same_bits(got[t], want[t], f"{name} position {t}")
    for st in (a, b):
        st.free()
    for mt in mats_a + mats_b:
        mt.free()
    assert dev.used == 0
