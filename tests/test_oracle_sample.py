"""Pins of the oracle's sampler (oracle/rk_oracle.c rko_sampler_*,
rko_sample; internal/llm/sample.go:11-43) by what the mathematics fixes,
not by retyping its steps:
* the state update is a linear map over GF(2)^64 of full period 2^64-1 (a
  dropped or wrong shift breaks one or the other);
* the draw is the top 24 bits of the scrambled state over 2^24, uniform;
* NewSampler's zero seed;
* r < cum is strict, on draws constructed to equal a cumulative sum exactly;
* the cumulative sum is float32 added in order (an accumulation in float64,
  or in another order, picks other tokens on long rows);
* the temperature divides the logits (the picks follow softmax(l/T));
* temperature <= 0 is the argmax and leaves the state; NaN samples.
"""
import numpy as np
import pytest

from oracle import oracle

MASK = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15
# Vigna's xorshift64* output multiplier ("An experimental exploration of
# Marsaglia's xorshift generators, scrambled", 2016)
MULT = 0x2545F4914F6CDD1D


def step(state):
    """The oracle's state update and draw: (new state, r)."""
    s = oracle.Sampler(1.0, state)
    r = s.next()
    return s.state.value, r


def gf2_apply(cols, v):
    out = 0
    i = 0
    while v:
        if v & 1:
            out ^= cols[i]
        v >>= 1
        i += 1
    return out


def gf2_mul(a, b):
    """Columns of a·b."""
    return [gf2_apply(a, c) for c in b]


def gf2_pow(m, e):
    r = [1 << i for i in range(64)]
    while e:
        if e & 1:
            r = gf2_mul(m, r)
        m = gf2_mul(m, m)
        e >>= 1
    return r


def test_state_update_is_a_full_period_linear_map():
    cols = [step(1 << i)[0] for i in range(64)]
    rng = np.random.default_rng(1)
    for _ in range(200):
        a, b = (int(x) for x in rng.integers(1, 1 << 63, 2, dtype=np.uint64))
        assert step(a ^ b)[0] == step(a)[0] ^ step(b)[0]
        assert step(a)[0] == gf2_apply(cols, a)
    ident = [1 << i for i in range(64)]
    primes = [3, 5, 17, 257, 641, 65537, 6700417]
    assert np.prod([float(p) for p in primes]) == float(MASK) and eval("*".join(map(str, primes))) == MASK
    assert gf2_pow(cols, MASK) == ident
    for p in primes:
        assert gf2_pow(cols, MASK // p) != ident, p


def test_draw_is_the_scrambled_states_top_24_bits():
    state = 12345
    rs = []
    for _ in range(2000):
        new, r = step(state)
        k = r * np.float32(1 << 24)
        assert k == np.floor(k) and 0 <= k < 1 << 24
        assert int(k) == ((new * MULT) & MASK) >> 40
        rs.append(r)
        state = new
    # uniform: a chi-square over 32 bins of 40000 draws
    s = oracle.Sampler(1.0, 99)
    r = np.array([s.next() for _ in range(40000)])
    h = np.histogram(r, bins=32, range=(0, 1))[0]
    chi2 = float(((h - 1250.0) ** 2 / 1250.0).sum())
    assert chi2 < 70, chi2  # 31 degrees of freedom: p < 2e-4 above 70


def test_zero_seed_is_replaced():
    assert oracle.Sampler(1.0, 0).state.value == GOLDEN
    assert oracle.Sampler(1.0, 5).state.value == 5
    assert oracle.Sampler(0.0, MASK).state.value == MASK


def unstep(x):
    """The state before `step` gave x (the three xorshifts undone)."""
    x ^= (x >> 27) ^ (x >> 54)
    x ^= ((x << 25) ^ (x << 50)) & MASK
    x ^= (x >> 12) ^ (x >> 24) ^ (x >> 36) ^ (x >> 48) ^ (x >> 60)
    return x


def seed_drawing(k):
    """A state whose next draw is exactly k / 2^24."""
    inv = pow(MULT, -1, 1 << 64)
    target = ((k << 40) + 1) * inv & MASK  # new state with (new·MULT) >> 40 == k (never 0)
    seed = unstep(target)
    assert step(seed) == (target, np.float32(k) / np.float32(1 << 24))
    return seed


def test_comparison_is_strict():
    two = np.array([0.0, 0.0], np.float32)
    assert list(oracle.sample_probs(two, 1.0)) == [0.5, 0.5]
    # r = 0.5 equals p0: not r < 0.5, the second token
    assert oracle.Sampler(1.0, seed_drawing(1 << 23)).sample(two) == 1
    assert oracle.Sampler(1.0, seed_drawing((1 << 23) - 1)).sample(two) == 0
    # r = 0 and a first probability of exactly 0: not 0 < 0
    lead0 = np.array([-200.0, 0.0, 0.0], np.float32)
    assert oracle.sample_probs(lead0, 1.0)[0] == 0.0
    assert oracle.Sampler(1.0, seed_drawing(0)).sample(lead0) == 1
    # r at the top: the last token
    assert oracle.Sampler(1.0, seed_drawing((1 << 24) - 1)).sample(two) == 1


def f32_pick(p, r):
    cum = np.add.accumulate(np.asarray(p, np.float32), dtype=np.float32)
    above = np.nonzero(r < cum)[0]
    return int(above[0]) if above.size else len(p) - 1


def test_cumulative_sum_is_float32_in_order():
    rng = np.random.default_rng(5)
    n = 100000
    differ = 0
    for trial in range(24):
        # a few distinct terms: float32 rounds each addition the same way
        # for long stretches, so its running sum drifts from the exact one
        logits = (rng.integers(0, 4, n) * 0.25).astype(np.float32)
        t = np.float32(0.9)
        seed = int(rng.integers(1, 1 << 62))
        p = oracle.sample_probs(logits, t)
        _, r = step(seed)
        got = oracle.Sampler(t, seed).sample(logits)
        assert got == f32_pick(p, r), trial
        c64 = np.cumsum(p.astype(np.float64))
        f64 = int(np.nonzero(r < c64)[0][0]) if (r < c64).any() else n - 1
        differ += f64 != got
    # the test can tell: a float64 running sum picks other tokens
    assert differ >= 12, differ


def test_temperature_divides_the_logits():
    logits = np.array([0.0, 1.0, 2.0, 3.0], np.float32)
    for t in (0.5, 2.0):
        s = oracle.Sampler(t, 77)
        n = 60000
        counts = np.bincount([s.sample(logits) for _ in range(n)], minlength=4)
        want = np.exp(logits / t) / np.exp(logits / t).sum() * n
        chi2 = float(((counts - want) ** 2 / want).sum())
        assert chi2 < 20, (t, counts, want)  # 3 degrees of freedom


def test_greedy_and_nan():
    logits = np.array([0.5, 3.0, 3.0, -1.0], np.float32)
    for t in (0.0, -0.0, -1.0, -np.inf):
        s = oracle.Sampler(t, 42)
        assert s.sample(logits) == 1
        assert s.state.value == 42  # the argmax draws nothing
    s = oracle.Sampler(np.nan, 42)
    assert s.sample(logits) == 3  # every probability NaN: the last token
    assert s.state.value == step(42)[0]
    s = oracle.Sampler(1.0, 42)
    assert s.sample(np.array([1.0, np.nan, 2.0], np.float32)) == 2
    assert s.state.value == step(42)[0]


def test_equal_logits_closed_form():
    """n equal logits: p_i = Recip32(n) each; the pick is the first i where
    r < (i+1)·p in float32 steps, about floor(r·n)."""
    for n in (3, 7, 10, 1000):
        logits = np.full(n, 0.25, np.float32)
        p = oracle.sample_probs(logits, 1.3)
        assert np.all(p == p[0]) and abs(float(p[0]) * n - 1) < 1e-6
        for seed in range(1, 60):
            _, r = step(seed)
            got = oracle.Sampler(1.3, seed).sample(logits)
            assert abs(got - int(r * n)) <= 1, (n, seed)
