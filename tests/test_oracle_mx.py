"""The CPU oracle of DeepSeek-V4.1's block-scaled arithmetic
(oracle/rk_oracle_mx.c, restating internal/num/mx.go) against the
reference's own vectors (tests/golden/dsv41-mx.json.gz, the reference
kernels' answers, as internal/num/mx_test.go:91-265 checks them) and
against closed forms: every E4M3 code's value and round trip, E8M0 and
E2M1 tables, the input quantization's scale rule, and products small
enough to sum by hand."""
import base64
import gzip
import json
import os

import numpy as np
import pytest

from oracle import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "dsv41-mx.json.gz")


@pytest.fixture(scope="module")
def vec():
    with gzip.open(GOLDEN, "rt") as f:
        return json.load(f)


def b64(s):
    return np.frombuffer(base64.b64decode(s), np.uint8)


def bf16s(s):
    return (b64(s).view("<u2").astype(np.uint32) << 16).view(np.float32)


def f32s(s):
    return b64(s).view("<f4").astype(np.float32)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_e4m3_codes():
    """mx_test.go:91-109: every non-NaN code round-trips, two NaNs,
    0x7e = 448, 0x01 = 2^-9, 0x38 = 1, saturation at ±1000."""
    v = oracle.e4m3_values()
    nan = np.isnan(v)
    assert nan.sum() == 2 and nan[0x7F] and nan[0xFF]
    codes = np.arange(256, dtype=np.uint8)
    assert np.array_equal(oracle.encode_e4m3(v[~nan].astype(np.float32)), codes[~nan])
    assert v[0x7E] == 448 and v[0x01] == 2.0 ** -9 and v[0x38] == 1 and v[0x08] == 2.0 ** -6
    assert list(oracle.encode_e4m3([1000, -1000, np.nan])) == [0x7E, 0xFE, 0x7F]
    # the grid: normal codes (8+m) 2^(e-10), subnormal m 2^-9
    for c in range(128):
        e, m = c >> 3, c & 7
        if c == 0x7F:
            continue
        want = m * 2.0 ** -9 if e == 0 else (8 + m) * 2.0 ** (e - 10)
        assert v[c] == want and v[c | 0x80] == -want


def test_encode_e4m3_matches_reference(vec):
    x = f32s(vec["round_e4m3"]["in"])
    want = b64(vec["round_e4m3"]["out"])
    got = oracle.encode_e4m3(x)
    assert np.array_equal(got, want), f"{int(np.sum(got != want))} of {x.size} differ"


def test_encode_e4m3_ties_to_even():
    """Halfway between two codes rounds to the even mantissa; below 2^-6
    the grid is 2^-9."""
    for c in range(1, 0x7E):
        lo, hi = oracle.e4m3_values()[c], oracle.e4m3_values()[c + 1]
        mid = np.float32((lo + hi) / 2)
        if float(mid) != (lo + hi) / 2:
            continue
        want = c if c % 2 == 0 else c + 1
        assert oracle.encode_e4m3([mid])[0] == want, hex(c)


def test_e8m0_and_e2m1_tables():
    L = oracle.lib()
    assert np.isnan(L.rko_decode_e8m0(255))
    assert np.float32(L.rko_decode_e8m0(0)) == np.float32(2.0 ** -127)
    for c in range(1, 255):
        assert L.rko_decode_e8m0(c) == 2.0 ** (c - 127)
    grid = [0, 0.5, 1, 1.5, 2, 3, 4, 6]
    for c in range(16):
        v = L.rko_decode_e2m1(c)
        assert abs(v) == grid[c & 7] and (np.signbit(v) == bool(c & 8))
    # every multiple of 1/64 in [-6, 6]: nearest, ties to the even code
    # (mx_test.go:127-148)
    for i in range(-6 * 64, 6 * 64 + 1):
        x = i / 64
        c = L.rko_encode_e2m1(x)
        d = [abs(abs(x) - g) for g in grid]
        best = min(d)
        cands = [k for k in range(8) if d[k] == best]
        want = cands[0] if len(cands) == 1 else [k for k in cands if k % 2 == 0][0]
        assert c & 7 == want and bool(c & 8) == (x < 0 or (x == 0 and np.signbit(x))), x


def test_act_quant_matches_reference(vec):
    """mx_test.go:161-187: codes, scale bytes and the in-place values."""
    for n, c in enumerate(vec["act_quant"]):
        x, q, sc, inplace = bf16s(c["x"]), b64(c["q"]), b64(c["scale"]), bf16s(c["inplace"])
        for r in range(c["rows"]):
            row = x[r * c["cols"]:(r + 1) * c["cols"]]
            codes, scales = oracle.act_fp8(row)
            assert np.array_equal(codes, q[r * c["cols"]:(r + 1) * c["cols"]]), f"case {n} row {r}"
            nb = c["cols"] // 32
            assert np.array_equal((bits(scales) >> 23).astype(np.uint8), sc[r * nb:(r + 1) * nb])
            got = oracle.act_quant_inplace(row)
            assert np.array_equal(bits(got), bits(inplace[r * c["cols"]:(r + 1) * c["cols"]]))


def test_act_scale_closed_form():
    """The scale is the least power of two s with amax / s <= 448 (amax
    floored at 1e-4), and a block holding 448 has s = 1."""
    rng = np.random.default_rng(3)
    for _ in range(200):
        x = (rng.normal(0, 1, 32) * 2.0 ** rng.integers(-30, 30)).astype(np.float32)
        _, s = oracle.act_fp8(x)
        amax = max(float(np.max(np.abs(x))), float(np.float32(1e-4)))
        t = float(np.float32(np.float32(amax) * np.float32(1 / 448)))
        k = int(np.ceil(np.log2(t)))
        assert s[0] == 2.0 ** k or (2.0 ** (k - 1) >= t and s[0] == 2.0 ** (k - 1))
    x = np.zeros(32, np.float32)
    x[0] = 448
    assert oracle.act_fp8(x)[1][0] == 1


def test_fp4_quant_matches_reference(vec):
    """mx_test.go:189-222: packed codes, scale bytes and in-place values,
    E8M0 (blocks of 32) and E4M3 (blocks of 16) scales."""
    for c in vec["fp4_quant"]:
        e4m3 = c["scale_kind"] == "e4m3"
        assert c["block"] == (16 if e4m3 else 32)
        x, packed, sc, inplace = bf16s(c["x"]), b64(c["packed"]), b64(c["scale"]), bf16s(c["inplace"])
        gp, gs = oracle.quantize_fp4(x, e4m3)
        assert np.array_equal(gs, sc), c["scale_kind"]
        assert np.array_equal(gp, packed), c["scale_kind"]
        got = oracle.dequant_fp4(gp, gs, x.size, e4m3)
        assert np.array_equal(bits(got), bits(inplace)), c["scale_kind"]


@pytest.mark.parametrize("kind", ["fp8_gemm", "fp4_gemm"])
def test_gemm_matches_reference(vec, kind):
    """mx_test.go:224-265: every output, rounded to bfloat16 and as the
    float32 sum before rounding (where the order of adding blocks shows)."""
    mv = oracle.matvec_fp8 if kind == "fp8_gemm" else oracle.matvec_fp4
    for c in vec[kind]:
        M, N, K = c["m"], c["n"], c["k"]
        x, w, ws = bf16s(c["x"]), b64(c["w"]), b64(c["w_scale"])
        y, y32 = bf16s(c["y"]), f32s(c["y32"])
        for r in range(M):
            xr = x[r * K:(r + 1) * K]
            got = mv(w, ws, xr, N, K, bf16=True)
            assert np.array_equal(bits(got), bits(y[r * N:(r + 1) * N])), f"{kind} {M}x{N}x{K} row {r}"
            got32 = mv(w, ws, xr, N, K, bf16=False)
            assert np.array_equal(bits(got32), bits(y32[r * N:(r + 1) * N])), f"{kind} {M}x{N}x{K} row {r} f32"


def test_fp8_sum_rounds_to_even():
    """internal/gpu/mx_test.go:180-238: block sums 2^25 + 2^18 + 2^17 - 1
    and - 2 (units of 2^-18) round to float32 first, then to bfloat16:
    130, never 2^25 + 2^18's 129."""
    cols = 32
    x = np.zeros(cols, np.float32)
    x[0] = x[1] = x[2] = 256
    x[3] = 2.0 ** -9
    rows = []
    for low in (0x81, 0x82):
        row = [int(oracle.encode_e4m3([0.5])[0]), 2, 1, low]
        rows.append(row)
        rows.append([b ^ 0x80 for b in row])
    w = np.zeros((len(rows), cols), np.uint8)
    for i, r in enumerate(rows):
        w[i, :4] = r
    got = oracle.matvec_fp8(w.ravel(), np.array([127], np.uint8), x, len(rows), cols)
    assert list(got) == [130, -130, 130, -130]


def test_fp8_tie_stays_even():
    """internal/gpu/mx_test.go:240-267: 128 + 2^-16 rounds to 128 in float32;
    then + 0.5 is a bfloat16 tie, down to 128."""
    cols = 64
    x = np.zeros(cols, np.float32)
    x[0], x[1], x[32] = 256, 2.0 ** -9, 256
    w = np.zeros(cols, np.uint8)
    w[0], w[1], w[32] = oracle.encode_e4m3([0.5])[0], 2, 1
    assert oracle.matvec_fp8(w, np.array([127, 127], np.uint8), x, 1, cols)[0] == 128


def test_fp8_exact_through_cancellation():
    """internal/gpu/mx_test.go:298-328: 15 products of 896, one of
    225 2^-13, 15 of -896: the block sum is exactly 225 2^-13."""
    cols = 32
    x = np.zeros(cols, np.float32)
    w = np.zeros(cols, np.uint8)
    x[0] = 448
    for i in range(1, 32):
        x[i], w[i] = 256, oracle.encode_e4m3([3.5])[0]
        if i > 16:
            w[i] |= 0x80
    x[16], w[16] = 0.9375, oracle.encode_e4m3([15.0 / 512])[0]
    got = oracle.matvec_fp8(w, np.array([127], np.uint8), x, 1, cols, bf16=False)
    assert got[0] == np.float32(225 * 2.0 ** -13)


def test_block_order_is_float32_in_order():
    """Blocks add in order in float32: 2^24, then 1, then -2^24 gives 0
    (1 is lost), while the other order would give 1."""
    cols = 96
    x = np.zeros(cols, np.float32)
    x[0] = 448
    x[32] = 448
    x[64] = 448
    w = np.zeros(cols, np.uint8)
    w[0] = w[64] = 0x7E  # 448
    w[64] |= 0x80
    w[32] = oracle.encode_e4m3([1 / 448.0 * 2 ** -6])[0]  # a tiny product
    ws = np.array([127 + 7, 127, 127 + 7], np.uint8)  # 448*448*128 ~ 2^24.6
    got = oracle.matvec_fp8(w, ws, x, 1, cols, bf16=False)[0]
    big = np.float32(np.float32(448.0 * 448.0) * np.float32(128))
    small = np.float32(oracle.e4m3_values()[w[32]] * 448)
    assert got == np.float32(np.float32(big + small) - big)
