"""The device sampler (rk_sample_logits, rk_stage_sampler) picks the
oracle's tokens and leaves the oracle's generator states, bit for bit
(internal/llm/sample.go:11-43):
* rows of logits at vocabulary sizes around the sampler's one-by-one prefix
  (256 terms) and its 16384-term scan chunks, up to 152064, from flat to
  peaked, with -inf, +inf and NaN logits, subnormal terms and terms spread
  over many binades (the exact scan's events: binade crossings and ties);
  temperatures from 1e-3 to 50, <= 0 (the argmax, no draw) and NaN; two
  picks in a row from each state;
* sampled generation inside the recorded step, one sequence and several
  (each with its own temperature and seed, one of them greedy), against the
  oracle's token loop with a Sampler (generate.go:446, :538), and back to
  greedy after.
"""
import numpy as np
import pytest

import rkhip
from oracle import oracle
from oracle.model import Config, Stage
from test_gpu_fused_stage import coded_model, oracle_generate, upload_layers

pytestmark = pytest.mark.gpu

GOLDEN = 0x9E3779B97F4A7C15


def oracle_pick(logits, temps, states):
    """Each row's pick and the state after it, by the oracle's Sampler."""
    toks, after = [], []
    for row, t, s in zip(logits, temps, states):
        smp = oracle.Sampler(t, int(s))
        toks.append(smp.sample(row))
        after.append(smp.state.value)
    return np.array(toks, np.int32), np.array(after, np.uint64)


def rows_for(kind, vocab, rng, n):
    if kind == "normal":
        return rng.normal(0, 2, (n, vocab)).astype(np.float32)
    if kind == "peaked":
        return (rng.normal(0, 1, (n, vocab)) * 12).astype(np.float32)
    if kind == "neginf":
        x = rng.normal(0, 1, (n, vocab)).astype(np.float32)
        x[rng.random((n, vocab)) < 0.3] = -np.inf
        return x
    if kind == "binades":
        # the first terms subnormal or tiny, then each stretch ~2^20 larger:
        # the running sum crosses binades inside the scan steps
        x = np.empty((n, vocab), np.float32)
        levels = [-100.0, -86.0, -72.0, -58.0, -44.0, -30.0, -16.0, -2.0]
        edges = np.linspace(0, vocab, len(levels) + 1).astype(int)
        for lv, a, b in zip(levels, edges[:-1], edges[1:]):
            x[:, a:b] = lv + rng.normal(0, 0.3, (n, b - a))
        return x
    if kind == "equal":
        return np.full((n, vocab), 0.75, np.float32)
    if kind == "specials":
        x = rng.normal(0, 1, (n, vocab)).astype(np.float32)
        x[0, vocab // 2] = np.nan
        if n > 1:
            x[1, vocab // 3] = np.inf
        return x
    raise ValueError(kind)


TEMPS = np.array([1.0, 0.7, 1e-3, 50.0, 0.0, -1.0, np.nan, 1.3], np.float32)

CASES = [(v, "normal") for v in (1, 2, 5, 255, 256, 257, 300, 16639, 16640, 16641, 33031)] + [
    (152064, "normal"), (32000, "peaked"), (20000, "neginf"), (151936, "binades"), (40000, "binades"),
    (100000, "equal"), (5000, "specials"), (128256, "peaked")]


@pytest.mark.parametrize("vocab,kind", CASES)
def test_sample_rows_match_oracle(dev, vocab, kind):
    rng = np.random.default_rng(vocab + len(kind))
    rows = len(TEMPS)
    logits = rows_for(kind, vocab, rng, rows)
    seeds = rng.integers(1, 1 << 63, rows, dtype=np.uint64)
    seeds[0] = GOLDEN  # NewSampler's replacement of a zero seed
    state = seeds.copy()
    want_state = seeds.copy()
    for k in range(2):
        print(f"vocab {vocab} {kind} pick {k}", flush=True)
        got = dev.sample_logits(logits, TEMPS, state)
        want, want_state = oracle_pick(logits, TEMPS, want_state)
        assert np.array_equal(got, want), f"{kind} {vocab}, pick {k}: {got} vs {want}"
        assert np.array_equal(state, want_state), f"{kind} {vocab}, pick {k}: states"
        logits = logits[:, ::-1].copy()  # another row order for the second pick


def test_sample_many_draws_one_row(dev):
    """Sixty picks in a row from one state, on a row whose picks spread."""
    rng = np.random.default_rng(8)
    row = rng.normal(0, 0.5, 50000).astype(np.float32)
    state = np.array([12345], np.uint64)
    smp = oracle.Sampler(0.9, 12345)
    for k in range(60):
        got = dev.sample_logits(row, [0.9], state)[0]
        assert got == smp.sample(row), k
        assert int(state[0]) == smp.state.value


def oracle_generate_sampled(m, prompt, steps, ctx, temperature, seed):
    """The coordinator's loop with a Sampler (generate.go:446, :538)."""
    st = Stage(m, ctx)
    smp = oracle.Sampler(temperature, seed)
    toks = list(prompt)
    for pos in range(len(prompt) + steps - 1):
        x = st.forward(m.embed_token(toks[pos]), pos)
        if pos + 1 >= len(prompt):
            toks.append(smp.sample(m.logits(x)))
    return toks[len(prompt):]


SAMPLE_CFG = Config(dim=64, hidden=128, layers=2, heads=4, kv_heads=2, vocab=20000, seq_len=64, dtype="q8_0")


def stage_for(dev, m, ctx, seqs=1):
    c = m.c
    layers, mats = upload_layers(dev, m)
    emb = dev.upload(m.embed.kind, m.embed.rows, m.embed.cols, m.embed.q, m.embed.scales)
    mats.append(emb)
    cos, sin = m.rope(ctx)
    st = rkhip.Stage(dev, c.dim, c.hidden, c.heads, c.kv_heads, ctx, layers, cos, sin, head_dim=c.head_dim,
                     norm_eps=float(c.eps()), qkv_bias=c.qkv_bias, qk_norm=c.qk_norm, seqs=seqs)
    st.set_head(emb, emb, m.rms_final)
    return st, mats


def test_stage_sampled_generation(dev):
    m = coded_model(SAMPLE_CFG, seed=11, scale_lo=1e-3, scale_hi=1e-2)
    ctx, steps = 48, 12
    prompt = [5, 17, 19999, 3, 0]
    st, mats = stage_for(dev, m, ctx)
    try:
        for t, seed in ((1.0, 0), (0.6, 987654321), (2.5, 42)):
            print(f"temperature {t} seed {seed}", flush=True)
            want = oracle_generate_sampled(m, prompt, steps, ctx, t, seed)
            st.sampler(t, seed)
            assert list(st.generate(prompt, steps)) == want, (t, seed)
            # the state moved on: set it again for the same tokens
            st.sampler(t, seed)
            st.generate_start(prompt)
            st.generate_run(len(prompt) - 1)
            for _ in range(steps):
                st.generate_run(1)
            assert list(st.tokens(len(prompt), steps)) == want, (t, seed, "one step a call")
        # back to greedy: the argmax loop again
        st.sampler(0.0, 0)
        want_g, _ = oracle_generate(m, prompt, steps, ctx)
        assert list(st.generate(prompt, steps)) == want_g
    finally:
        st.free()
        for mt in mats:
            mt.free()
    assert dev.used == 0


def test_stage_sequences_sample_each_their_own(dev):
    m = coded_model(SAMPLE_CFG, seed=12, scale_lo=1e-3, scale_hi=1e-2)
    ctx, steps = 48, 10
    rng = np.random.default_rng(4)
    prompts = [[int(t) for t in rng.integers(0, SAMPLE_CFG.vocab, n)] for n in (1, 6, 3, 9)]
    samplers = [(1.0, 7), (0.0, 0), (0.8, 0), (1.7, 123456789)]
    st, mats = stage_for(dev, m, ctx, seqs=len(prompts))
    try:
        for z, (t, seed) in enumerate(samplers):
            st.sampler(t, seed, seq=z)
        st.seqs_start(prompts)
        st.seqs_run(steps)
        for z, (p, (t, seed)) in enumerate(zip(prompts, samplers)):
            want = oracle_generate_sampled(m, p, steps, ctx, t, seed)
            assert list(st.seqs_tokens(z, len(p), steps)) == want, (z, t, seed)
    finally:
        st.free()
        for mt in mats:
            mt.free()
    assert dev.used == 0
