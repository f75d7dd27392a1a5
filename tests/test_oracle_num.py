"""Pins the CPU oracle's restatement of internal/num before it is trusted.

Each check is one the reference itself holds (its known answers, digests and
error bounds), an invariant of the algorithm, or a closed form chosen so that
a plausible slip (a dropped rounding, a reordered sum, a wrong constant)
fails it. Paths in citations are relative to the rakkan-mesh repository.
"""
import json
import math
import os
import re
from fractions import Fraction
from decimal import Decimal

import numpy as np
import pytest

from oracle import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_known_answers.json")))


def bits(v):
    return int(np.float32(v).view(np.uint32))


def f32_round(fr: Fraction) -> int:
    """Bits of the float32 nearest to the exact rational fr (ties to even)."""
    sign = 0x80000000 if fr < 0 else 0
    fr = abs(fr)
    e = fr.numerator.bit_length() - fr.denominator.bit_length()
    while Fraction(2) ** e > fr:
        e -= 1
    while Fraction(2) ** (e + 1) <= fr:
        e += 1
    m = fr / Fraction(2) ** (e - 23)
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign | int(np.float32(float(Fraction(fl) * Fraction(2) ** (e - 23))).view(np.uint32))


# --- the reference's own digest ----------------------------------------------

def test_transcendental_digest_matches_reference():
    """internal/num/num_test.go:351-376: 100000 steps of Go's PCG(9,10)
    stream through Log, Log1p, Exp32 and Sincos, hashed. Pins the Go RNG
    (PCG-DXSM, Float64, IntN) and all four functions bit for bit."""
    g = GOLD["transcendental_digest"]
    assert oracle.transcendental_digest(g["steps"]) == g["sha256"]


# --- float32 constants ---------------------------------------------------------

CONSTS = {
    "1_127": Fraction(1, 127), "24_17": Fraction(24, 17), "8_17": Fraction(8, 17),
    "LOG2E": Fraction(Decimal("1.4426950408889634")), "LN2HI": Fraction(Decimal("0.693145751953125")),
    "LN2LO": Fraction(Decimal("1.428606765330187e-06")), "1_720": Fraction(1, 720), "1_120": Fraction(1, 120),
    "1_24": Fraction(1, 24), "1_6": Fraction(1, 6), "EXP_HI": Fraction(Decimal("88.72")),
    "EXP_LO": Fraction(Decimal("-103.97")),
}


def test_constants_are_go_roundings():
    """Go rounds an untyped constant once to float32; the oracle and the HIP
    kernels write those constants as bit patterns. Re-derive each from the
    exact rational and compare with both sources."""
    src = open(os.path.join(ROOT, "oracle", "rk_oracle.c")).read()
    for name, fr in CONSTS.items():
        m = re.search(r"#define K_%s\s+0x([0-9a-f]+)u" % name, src)
        assert m, name
        assert int(m.group(1), 16) == f32_round(fr), name
    dev = open(os.path.join(ROOT, "rakkan-mesh_amd", "csrc", "rk_fmath.h")).read()
    dev_names = {"1_127": "k1_127", "24_17": "k24_17", "8_17": "k8_17", "LOG2E": "kLog2e", "LN2HI": "kLn2Hi",
                 "LN2LO": "kLn2Lo", "EXP_HI": "kExpHi", "EXP_LO": "kExpLo"}
    for name, cname in dev_names.items():
        m = re.search(r"constexpr uint32_t %s = 0x([0-9a-f]+)u" % cname, dev)
        assert m, cname
        assert int(m.group(1), 16) == f32_round(CONSTS[name]), cname


def test_float64_constants():
    """math.Sqrt2/2 (Log) and 2/math.Pi (Sincos) are exact expressions of Go's
    long decimal constants, rounded once to float64."""
    sqrt2 = Fraction(Decimal("1.41421356237309504880168872420969807856967187537694807317667974"))
    pi = Fraction(Decimal("3.14159265358979323846264338327950288419716939937510582097494459"))
    assert float(sqrt2 / 2) == 0.70710678118654752440
    assert float(2 / pi) == 0.63661977236758134308


# --- Recip32, Rsqrt32, Exp32 ---------------------------------------------------

def test_recip_rsqrt_known_answers():
    """internal/num/num_test.go:319-325."""
    for x, want in GOLD["recip_rsqrt_exact"]["recip32"]:
        assert oracle.recip32(x) == want
    for x, want in GOLD["recip_rsqrt_exact"]["rsqrt32"]:
        assert oracle.rsqrt32(x) == want
    inf = np.float32(np.inf)
    assert oracle.recip32(0.0) == inf and oracle.recip32(inf) == 0
    assert oracle.rsqrt32(0.0) == inf and oracle.rsqrt32(inf) == 0
    assert bits(oracle.recip32(-0.0)) == bits(-inf)
    assert bits(oracle.recip32(np.nan)) == 0x7FC00000
    assert bits(oracle.rsqrt32(-1.0)) == 0x7FC00000


def test_recip_rsqrt_within_two_ulp():
    """internal/num/num_test.go:274-318: over normal, arbitrary-bit, [0.25,4]
    and subnormal inputs, both within 2 ulp, Recip32(-x) = -Recip32(x), and
    Recip32 overflows to +Inf exactly when 1/x does."""
    rng = np.random.default_rng(5)
    n = 40000
    xs = np.concatenate([
        np.exp(rng.random(n) * 170 - 85).astype(np.float32),
        (rng.integers(0, 1 << 31, n, dtype=np.uint64).astype(np.uint32) & 0x7F7FFFFF).view(np.float32),
        (rng.random(n) * 4 + 0.25).astype(np.float32),
        rng.integers(1, 1 << 23, n, dtype=np.uint32).view(np.float32),
    ])
    xs = xs[np.isfinite(xs) & (xs > 0)]
    worst_r = worst_s = 0.0
    for x in xs:
        x = np.float32(x)
        exact = 1.0 / float(x)
        r = oracle.recip32(x)
        if exact > float(np.finfo(np.float32).max):
            assert np.isinf(r)
        else:
            step = float(np.spacing(np.float32(exact))) or float(np.finfo(np.float32).smallest_subnormal)
            worst_r = max(worst_r, abs(float(r) - exact) / step)
        assert bits(oracle.recip32(-x)) == bits(-r)
        e2 = 1.0 / math.sqrt(float(x))
        step = float(np.spacing(np.float32(e2)))
        worst_s = max(worst_s, abs(float(oracle.rsqrt32(x)) - e2) / step)
    assert worst_r <= 2 and worst_s <= 2, (worst_r, worst_s)


def test_exp32_relative_error():
    """internal/num/num_test.go:49-58: relative error below 4e-7 on
    [-100, 88) in steps of 0.0137; the cut-offs of num.go:79-83."""
    worst = 0.0
    x = np.float32(-100)
    step = np.float32(0.0137)
    while x < 88:
        got, want = float(oracle.exp32(x)), math.exp(float(x))
        if want > 1e-37:
            worst = max(worst, abs(got - want) / want)
        x = np.float32(x + step)
    assert worst < 4e-7
    assert np.isinf(oracle.exp32(88.73)) and oracle.exp32(-104.0) == 0
    assert oracle.exp32(0.0) == 1.0
    assert bits(oracle.exp32(np.nan)) == 0x7FC00000


def test_go_float64_functions_close_to_libm():
    """internal/num/num_test.go:20-59, 328-346: Exp within 4 ulp, Log and
    Log1p within 2 ulp, Sincos within 4 ulp (absolute near zeros)."""
    L = oracle.lib()
    rng = np.random.default_rng(7)

    def ulps(a, b):
        return 0.0 if a == b else abs(a - b) / abs(math.nextafter(b, math.inf) - b)

    worst = 0.0
    for x in np.arange(-700.0, 700.0, 0.731):
        worst = max(worst, ulps(L.rko_exp(x), math.exp(x)))
    assert worst <= 4
    worst = 0.0
    for _ in range(20000):
        x = math.ldexp(1 + rng.random(), int(rng.integers(0, 200)) - 100)
        worst = max(worst, ulps(L.rko_log(x), math.log(x)))
        y = math.ldexp(rng.random(), -int(rng.integers(0, 60)))
        worst = max(worst, ulps(L.rko_log1p(y), math.log1p(y)))
    assert worst <= 2
    import ctypes
    s, c = ctypes.c_double(), ctypes.c_double()
    worst = 0.0
    for x in np.arange(-300.0, 300.0, 0.0731):
        L.rko_sincos(x, ctypes.byref(s), ctypes.byref(c))
        ws, wc = math.sin(x), math.cos(x)
        if abs(ws) > 1e-3:
            worst = max(worst, ulps(s.value, ws))
        else:
            assert abs(s.value - ws) <= 1e-15
        if abs(wc) > 1e-3:
            worst = max(worst, ulps(c.value, wc))
        else:
            assert abs(c.value - wc) <= 1e-15
    assert worst <= 4


def test_exp_within_one_ulp_of_correctly_rounded():
    """internal/num/num.go:101-123 Exp (float64; used for NewRope's
    frequencies). The reference pins it to 4 ulp of math.Exp (num_test.go:
    41-47); its Taylor series to r^13 over |r| <= 0.347 keeps it within one
    ulp of the correctly rounded value (50-digit Decimal), which a dropped
    ln2Lo term, a missing Taylor term or a wrong factorial would break. Bits
    beyond that are not pinned. Also its cut-offs (num.go:102-109)."""
    from decimal import getcontext

    getcontext().prec = 50
    L = oracle.lib()
    rng = np.random.default_rng(8)
    xs = [float(v) for v in np.arange(-700.0, 700.0, 1.37)] + [float(v) for v in rng.uniform(-40, 40, 2000)]
    xs += [k * math.log(2) for k in range(-60, 60)] + [math.nextafter(0.5 * math.log(2), 1.0)]
    exact = 0
    for x in xs:
        got, cr = L.rko_exp(x), float(Decimal(x).exp())
        if got != cr:
            assert abs(got - cr) <= abs(math.nextafter(cr, math.inf) - cr), (x, got, cr)
        else:
            exact += 1
    assert exact > 0.8 * len(xs)
    assert L.rko_exp(0.0) == 1.0 and math.isinf(L.rko_exp(709.79)) and L.rko_exp(-745.14) == 0.0
    assert math.isnan(L.rko_exp(math.nan))


def test_bf16_rounding():
    """internal/num/num_test.go:104."""
    L = oracle.lib()
    for x, want in GOLD["bf16"]["to_bf16"]:
        assert L.rko_to_bf16(np.float32(x)) == want


# --- Q8_0 / Q4_0 --------------------------------------------------------------

def test_quantize8_closed_forms():
    """internal/num/quant.go:34-53. A zero block gets scale 0 and zero codes;
    the largest magnitude maps to ±127; codes stay in [-127, 127] (never
    -128); dequantized values are within half a step."""
    w = np.zeros(96, np.float32)
    w[32:64] = np.linspace(-1, 1, 32, dtype=np.float32)
    w[64:96] = np.float32(1e-30) * np.arange(32, dtype=np.float32)
    q, s = oracle.quantize8(w)
    assert s[0] == 0 and not q[:32].any()
    assert q[32] == -127 and q[63] == 127
    assert s[1] == np.float32(np.float32(1.0) * np.float32(1.0 / 127))
    rng = np.random.default_rng(3)
    w = (rng.normal(0, 0.05, 300 * 896)).astype(np.float32)
    q, s = oracle.quantize8(w)
    assert q.min() >= -127 and q.max() <= 127
    deq = q.astype(np.float32) * np.repeat(s, 32)
    assert np.all(np.abs(deq - w) <= s.repeat(32) * 0.5001)


def test_quantize8_rounds_half_to_even():
    """internal/num/quant.go:41-50: codes are RoundToEven(v·id). With a
    block maximum of 127, d = 127·float32(1/127) is exactly 1 and
    Recip32(1) = 1, so v·id = v and the halves are ties: ±0.5, ±1.5, ±2.5,
    3.5 must give 0, ±2, ±2, 4. Rounding half away from zero gives ±1, ±2,
    ±3, 4; truncation 0, ±1, ±2, 3."""
    assert np.float32(127) * np.float32(1.0 / 127) == np.float32(1)
    assert oracle.recip32(1.0) == 1.0
    blk = np.zeros(32, np.float32)
    ties = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5, 126.5]
    blk[0] = 127
    blk[1:1 + len(ties)] = ties
    q, s = oracle.quantize8(blk)
    assert bits(s[0]) == bits(1.0)
    assert q[0] == 127
    assert list(q[1:1 + len(ties)]) == [0, 0, 2, -2, 2, -2, 4, 126]


def test_quantize8_multiplies_by_recip32_not_divides():
    """internal/num/quant.go:41: id = Recip32(d), then float32(v·id); no
    division. At d = float32(102.8525·float32(1/127)) = 0.8098622,
    Recip32(d) (0x3f9e0d35) is one ulp above the correctly rounded 1/d
    (0x3f9e0d34), and at these three inputs that ulp moves v·id across a
    rounding point: the exact products, rounded to float32, are 0.50000006,
    1.5 (a tie, to even: 2) and 2.5000002, giving codes 1, 2, 3; v/d gives
    0.5, 1.4999999 and 2.5 (codes 0, 1, 2), and v·float32(1/d) the same."""
    amax = np.uint32(0x42CDB47B).view(np.float32)
    d = np.float32(amax * np.float32(1.0 / 127))
    r = np.float32(oracle.recip32(d))
    assert bits(r) == 0x3F9E0D35 and bits(np.float32(1) / d) == 0x3F9E0D34
    vs = np.array([0x3ECF5321, 0x3F9B7E58, 0x400193F5], np.uint32).view(np.float32)
    blk = np.zeros(32, np.float32)
    blk[0] = amax
    blk[1:4] = vs
    blk[4:7] = -vs
    q, s = oracle.quantize8(blk)
    assert bits(s[0]) == bits(d)
    # the products rounded to float32, from exact rationals (not float code)
    prods = [f32_round(Fraction(float(v)) * Fraction(float(r))) for v in vs]
    assert prods == [bits(0.50000006), bits(1.5), bits(2.5000002)]
    assert list(q[1:7]) == [1, 2, 3, -1, -2, -3]


def test_quantized_matvec_error_bounds():
    """internal/num/num_test.go:167-206 (TestQuantized): against the f32
    product, Q8_0 within 1 % and Q4_0 within 15 % (relative L2); Q4_0 codes
    dequantize within two steps."""
    rng = np.random.default_rng(4)
    rows, cols = 300, 896
    w = rng.normal(0, 0.05, rows * cols).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    exact = oracle.matvec32(w, x, rows, cols)
    q8, s8 = oracle.quantize8(w)
    q4, s4 = oracle.quantize4(w)
    g8 = oracle.matvec_q8(q8, s8, x, rows, cols)
    g4 = oracle.matvec_q4(q4, s4, x, rows, cols)
    norm = np.sqrt(np.sum(exact.astype(np.float64) ** 2))
    e8 = np.sqrt(np.sum((g8 - exact).astype(np.float64) ** 2)) / norm
    e4 = np.sqrt(np.sum((g4 - exact).astype(np.float64) ** 2)) / norm
    assert e8 <= 0.01 and e4 <= 0.15, (e8, e4)
    d4 = np.empty(rows * cols, np.float32)
    oracle.lib().rko_dequant4(oracle.ptr(d4), oracle.ptr(q4), oracle.ptr(s4), rows * cols)
    assert np.all(np.abs(d4 - w) <= np.abs(s4.repeat(32)) * 2.0001 + 1e-9)


def test_block_sums_brute_force():
    """Exact integer block sums (quant.go:198-218) against int64 numpy, with
    the ±127 extremes of num_test.go:207-218, at 28, 27, 3 and 1 blocks."""
    rng = np.random.default_rng(11)
    L = oracle.lib()
    for nb in (28, 27, 3, 1):
        n = nb * 32
        w = rng.integers(-127, 128, n).astype(np.int8)
        w[::7] = 127
        w[::11] = -127
        x = rng.integers(-127, 128, n).astype(np.int8)
        got = np.empty(nb, np.int32)
        L.rko_blocksums_q8(oracle.ptr(w), oracle.ptr(x), nb, oracle.ptr(got))
        want = (w.astype(np.int64) * x.astype(np.int64)).reshape(nb, 32).sum(1)
        assert np.array_equal(got, want)
        # Q4: byte j = (v_j+8) | (v_{j+16}+8)<<4
        v = rng.integers(-8, 8, n).astype(np.int64).reshape(nb, 32)
        packed = ((v[:, :16] + 8) | ((v[:, 16:] + 8) << 4)).astype(np.uint8).ravel()
        L.rko_blocksums_q4(oracle.ptr(packed), oracle.ptr(x), nb, oracle.ptr(got))
        assert np.array_equal(got, (v * x.astype(np.int64).reshape(nb, 32)).sum(1))


def _qrow(sums, ws, xs):
    L = oracle.lib()
    sums, ws, xs = (np.ascontiguousarray(sums, np.int32), np.ascontiguousarray(ws, np.float32),
                    np.ascontiguousarray(xs, np.float32))
    return np.float32(L.rko_qrow(oracle.ptr(sums), oracle.ptr(ws), oracle.ptr(xs), sums.size))


def test_qrow_order_closed_form():
    """quant.go:14-19: block b goes to running sum b mod 8, in order, and the
    sums combine ((0+1)+(2+3))+((4+5)+(6+7)). With nine unit scales and block
    sums [2^24, 1 x 8]: sum 0 is 2^24 + 1 = 2^24 (the tie rounds to even),
    sums 1..7 are 1, so the tree gives ((2^24 + 1) + 2) + 4 = 2^24 + 6.
    A single sequential chain, or the eight sums added left to right, would
    lose every 1 and give 2^24."""
    sums = np.array([1 << 24] + [1] * 8, np.int32)
    got = _qrow(sums, np.ones(9, np.float32), np.ones(9, np.float32))
    assert got == np.float32(2 ** 24 + 6)
    # The scale product is rounded to float32 before the integer multiplies
    # it: ws·xs = (1+2^-12)^2 rounds to 1+2^-11, and 3·(1+2^-11) is exact;
    # unrounded it would be 3 + 6·2^-12 + 3·2^-24 -> rounds differently.
    a = np.float32(1 + 2 ** -12)
    got = _qrow(np.array([3], np.int32), np.array([a]), np.array([a]))
    assert got == np.float32(3 * (1 + 2 ** -11))


def test_avx2_path_equals_portable_and_split_invariant():
    """The CPU baseline (AVX2 block sums, rows split over threads) gives the
    portable oracle's bits: num_test.go:61-81 (split independence) and
    207-232 (vector = portable)."""
    if not oracle.lib().rko_have_avx2():
        pytest.skip("no AVX2 on this host")
    rng = np.random.default_rng(12)
    for rows, cols in ((7, 32), (300, 896), (64, 4864), (1000, 96), (513, 288)):
        q = rng.integers(-127, 128, rows * cols).astype(np.int8)
        q[::13] = 127
        q[::17] = -127
        s = rng.uniform(1e-3, 1e-2, rows * cols // 32).astype(np.float32)
        x = rng.normal(0, 1, cols).astype(np.float32)
        want = oracle.matvec_q8(q, s, x, rows, cols)
        for th in (1, 3, 8):
            got = oracle.matvec_q8_avx2(q, s, x, rows, cols, th)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        q4 = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
        want4 = oracle.matvec_q4(q4, s, x, rows, cols)
        got4 = oracle.matvec_q4_avx2(q4, s, x, rows, cols, 5)
        assert np.array_equal(got4.view(np.uint32), want4.view(np.uint32))


def test_rows_are_independent():
    """Each row is one computation (quant.go:173-179): permuting rows
    permutes the outputs bit for bit."""
    rng = np.random.default_rng(13)
    rows, cols = 64, 4864
    q = rng.integers(-127, 128, rows * cols).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, rows * cols // 32).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    base = oracle.matvec_q8(q, s, x, rows, cols)
    perm = rng.permutation(rows)
    qp = q.reshape(rows, cols)[perm].ravel()
    sp = s.reshape(rows, cols // 32)[perm].ravel()
    got = oracle.matvec_q8(qp, sp, x, rows, cols)
    assert np.array_equal(got.view(np.uint32), base[perm].view(np.uint32))


def test_activation_quantize_equals_weight_quantize():
    """QuantizeActs and QuantizeQ8 are the same function (quant.go:150-156),
    and the matvec quantizes its input exactly so: the product equals integer
    block sums of the quantized input combined with its scales."""
    rng = np.random.default_rng(14)
    rows, cols = 16, 96
    q = rng.integers(-127, 128, rows * cols).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, rows * cols // 32).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    qx, xs = oracle.quantize8(x)
    L = oracle.lib()
    sums = np.empty(3, np.int32)
    for r in range(rows):
        L.rko_blocksums_q8(oracle.ptr(np.ascontiguousarray(q[r * cols:(r + 1) * cols])), oracle.ptr(qx), 3,
                           oracle.ptr(sums))
        want = _qrow(sums, s[r * 3:(r + 1) * 3], xs)
        assert bits(oracle.matvec_q8(q[r * cols:(r + 1) * cols], s[r * 3:(r + 1) * 3], x, 1, cols)[0]) == bits(want)


def test_dot32_order_closed_forms():
    """Dot32 (internal/num/matvec.go:32-67): each input pins one part of the
    order, because the plausible alternative gives another float32.
    * a running sum adds its elements in order: 1e8 + 1 rounds back to 1e8,
      so s0 = ((1e8 + 1) - 1e8) is 0 (another order gives 1);
    * e_j = (s_j + s_j+8) + (s_j+16 + s_j+24): with s0 = 1e8, s8 = -1e8,
      s16 = 1 it is 1 ((s0 + s16) + (s8 + s24) gives 0);
    * ((e0+e1)+(e2+e3))+((e4+e5)+(e6+e7)): with e0 = 1, e2 = 1e8,
      e3 = -1e8 it is 1 (a left fold gives 0), and with e4 = 1e8,
      e5 = -1e8, e6 = 1 likewise;
    * each product is rounded before it is added (no fused multiply-add):
      (1+2^-12)^2 rounds to 1+2^-11, so adding -(1+2^-11) gives 0 (2^-24
      with a fused multiply-add)."""
    def d(a, b=None):
        a = np.asarray(a, np.float32)
        return oracle.dot32(a, np.ones_like(a) if b is None else np.asarray(b, np.float32))

    a = np.zeros(96, np.float32)
    a[0], a[32], a[64] = 1e8, 1, -1e8
    assert d(a) == 0.0
    a = np.zeros(32, np.float32)
    a[0], a[8], a[16] = 1e8, -1e8, 1
    assert d(a) == 1.0
    a = np.zeros(32, np.float32)
    a[0], a[2], a[3] = 1, 1e8, -1e8
    assert d(a) == 1.0
    a = np.zeros(32, np.float32)
    a[4], a[5], a[6] = 1e8, -1e8, 1
    assert d(a) == 1.0
    u = np.float32(1 + 2.0 ** -12)
    a = np.zeros(64, np.float32)
    b = np.ones(64, np.float32)
    a[0], b[0], a[32] = u, u, -np.float32(1 + 2.0 ** -11)
    assert d(a, b) == 0.0
    # all partial sums exact: the integer dot product, any length (tails too)
    rng = np.random.default_rng(11)
    for n in (1, 31, 33, 100, 4097):
        ai = rng.integers(-50, 51, n)
        bi = rng.integers(-50, 51, n)
        assert d(ai.astype(np.float32), bi.astype(np.float32)) == float(np.dot(ai, bi))


def test_dot_bf16_equals_dot32_and_error_bound():
    """internal/num/num_test.go:83-105 (TestDot8AndBF16): DotBF16 equals
    Dot32 on the converted weights bit for bit, and Dot32 is within
    1e-4·sqrt(n) + 1e-6 of the exact product."""
    rng = np.random.default_rng(2)
    for n in (0, 1, 7, 8, 9, 63, 896, 4865):
        w16 = oracle.to_bf16(rng.normal(0, 1, n).astype(np.float32))
        w = (w16.astype(np.uint32) << 16).view(np.float32)  # BF16: the upper half of a float32
        x = rng.normal(0, 1, n).astype(np.float32)
        a, b = oracle.dot32(w, x), oracle.dot_bf16(w16, x)
        assert bits(a) == bits(b), n
        exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
        assert abs(float(a) - exact) <= 1e-4 * math.sqrt(n) + 1e-6, n


def test_matvec32_rows_are_dot32():
    """MatVec32 / MatVecBF16 (internal/num/matvec.go:106-123): row i is
    Dot32 of row i, whatever the split over workers."""
    rng = np.random.default_rng(5)
    rows, cols = 37, 300
    w = rng.normal(0, 1, rows * cols).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    got = oracle.matvec32(w, x, rows, cols)
    for i in range(rows):
        assert bits(got[i]) == bits(oracle.dot32(w[i * cols:(i + 1) * cols], x))
    w16 = oracle.to_bf16(w)
    got = oracle.matvec_bf16(w16, x, rows, cols)
    for i in range(rows):
        assert bits(got[i]) == bits(oracle.dot_bf16(w16[i * cols:(i + 1) * cols], x))
