"""DeepSeek-V4.1 block-scaled products on the GPU (internal/gpu/mx.go,
internal/num/mx.go): E4M3 (FP8) and packed E2M1 (FP4) weights with E8M0
scales, the input quantized on the device to E4M3 with power-of-two block
scales. Every output is compared bit for bit with the CPU oracle (itself
pinned to the reference kernels' vectors in test_oracle_mx.py), rounded to
bfloat16 and as the float32 sums before rounding; the reference's own
vectors run through the GPU too, and the cases of internal/gpu/mx_test.go
(rounding to even, ties, cancellation, large matrices, the batch path)."""
import base64
import gzip
import json
import os

import numpy as np
import pytest

import rkhip
from oracle import oracle

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "dsv41-mx.json.gz")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same_bits(got, want, what):
    g, w = bits(got), bits(want)
    if not np.array_equal(g, w):
        i = int(np.argmax(g != w))
        raise AssertionError(f"{what}: row {i}: GPU {got[i]!r} ({g[i]:#x}), oracle {want[i]!r} ({w[i]:#x}), "
                             f"{int(np.sum(g != w))} rows differ")


def random_fp8(rng, rows, cols):
    """Every code but the NaNs; scales around 1, some large, some at the
    subnormal end (mx_test.go:13-45 randomFP8 / randomScales)."""
    w = rng.integers(0, 256, rows * cols).astype(np.uint8)
    bad = (w & 0x7F) == 0x7F
    w[bad] = rng.integers(0, 0x7F, int(bad.sum())).astype(np.uint8) | (w[bad] & 0x80)
    return w, random_scales(rng, (rows + 31) // 32 * (cols // 32))


def random_scales(rng, n):
    pick = rng.integers(0, 20, n)
    s = rng.integers(110, 140, n)
    s[pick == 2] = rng.integers(200, 230, int((pick == 2).sum()))
    s[pick == 0] = 0                                      # 2^-127
    s[pick == 1] = rng.integers(1, 11, int((pick == 1).sum()))  # terms reaching denormals
    return s.astype(np.uint8)


def mx_input(rng, n, specials=False):
    """mx_test.go:47-83 mxInput: blocks all zero, huge, tiny, at E4M3
    rounding ties, or ordinary with denormals and signed zeros; with
    specials, also blocks holding an infinity or a NaN."""
    x = np.zeros(n, np.float32)
    for b in range(0, n, 32):
        k = rng.integers(0, 8 if specials else 6)
        blk = x[b:b + 32]
        if k == 0:
            pass
        elif k == 1:
            blk[:] = rng.normal(0, 1, 32) * 1e30
        elif k == 2:
            blk[:] = rng.normal(0, 1, 32) * 1e-6
        elif k == 3:
            blk[0] = 448
            e = rng.integers(0, 12, 31) - 3
            v = np.ldexp(8 + rng.integers(0, 8, 31) + 0.5, e - 3)
            blk[1:] = np.where(rng.integers(0, 2, 31) == 0, -v, v)
        elif k in (4, 5):
            blk[:] = rng.normal(0, 3, 32)
            pick = rng.integers(0, 40, 32)
            blk[pick == 0] = rng.integers(0, 1 << 23, int((pick == 0).sum()), dtype=np.uint32).view(np.float32)
            blk[pick == 1] = np.float32(-0.0)
            blk[pick == 2] = np.float32(1e-30)
        elif k == 6:
            blk[:] = rng.normal(0, 3, 32)
            blk[rng.integers(0, 32)] = np.inf if rng.integers(0, 2) else -np.inf
        else:
            blk[:] = rng.normal(0, 3, 32)
            blk[rng.integers(0, 32)] = np.nan
    return x


def check_both(dev, m, x, cpu):
    """The product rounded to bfloat16, then left in float32."""
    same_bits(dev.matvecs([m], x)[0], cpu(True), "bf16")
    m.set_raw(True)
    try:
        same_bits(dev.matvecs([m], x)[0], cpu(False), "float32")
    finally:
        m.set_raw(False)


def b64(s):
    return np.frombuffer(base64.b64decode(s), np.uint8)


def bf16s(s):
    return (b64(s).view("<u2").astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("kind", ["fp8_gemm", "fp4_gemm"])
def test_reference_vectors_on_gpu(dev, kind):
    """The reference kernels' answers (internal/num/testdata/dsv41-mx.json.gz)
    from the GPU: bfloat16 results and float32 sums."""
    with gzip.open(GOLDEN, "rt") as f:
        cases = json.load(f)[kind]
    fmt = rkhip.FP8 if kind == "fp8_gemm" else rkhip.FP4
    for c in cases:
        M, N, K = c["m"], c["n"], c["k"]
        x, w, ws = bf16s(c["x"]), b64(c["w"]), b64(c["w_scale"])
        y, y32 = bf16s(c["y"]), b64(c["y32"]).view("<f4")
        print(f"{kind} {M}x{N}x{K}", flush=True)
        m = dev.upload_mx(fmt, N, K, w, ws)
        try:
            for r in range(M):
                xr = x[r * K:(r + 1) * K]
                same_bits(dev.matvecs([m], xr)[0], y[r * N:(r + 1) * N], f"{kind} {M}x{N}x{K} row {r}")
                m.set_raw(True)
                same_bits(dev.matvecs([m], xr)[0], y32[r * N:(r + 1) * N], f"{kind} {M}x{N}x{K} row {r} f32")
                m.set_raw(False)
        finally:
            m.free()
    assert dev.used == 0


SHAPES = [(7, 32), (33, 64), (300, 896), (64, 5120), (1000, 96), (40, 2304), (17, 1280), (100, 18432), (5, 40000)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_fp8_matches_cpu(dev, rows, cols):
    rng = np.random.default_rng(rows * 131 + cols)
    x = mx_input(rng, cols, specials=True)
    w, s = random_fp8(rng, rows, cols)
    m = dev.upload_mx(rkhip.FP8, rows, cols, w, s)
    try:
        check_both(dev, m, x, lambda r: oracle.matvec_fp8(w, s, x, rows, cols, bf16=r))
    finally:
        m.free()
    assert dev.used == 0


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_fp4_matches_cpu(dev, rows, cols):
    rng = np.random.default_rng(rows * 137 + cols)
    x = mx_input(rng, cols, specials=True)
    w = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    s = random_scales(rng, rows * cols // 32)
    m = dev.upload_mx(rkhip.FP4, rows, cols, w, s)
    try:
        check_both(dev, m, x, lambda r: oracle.matvec_fp4(w, s, x, rows, cols, bf16=r))
    finally:
        m.free()
    assert dev.used == 0


def test_fp4_infinite_input_block(dev):
    """An input block with infinities has scale +inf and NaN codes where the
    infinities were; the CPU's integer sum then holds 0x80000000 for each
    odd twice-weight there (Go's int32(NaN) on x86-64): -inf or NaN terms."""
    cols, rows = 64, 64
    x = np.ones(cols, np.float32)
    x[3] = np.inf
    x[9] = -np.inf
    x[40] = np.nan
    rng = np.random.default_rng(4)
    w = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    s = np.full(rows * cols // 32, 127, np.uint8)
    m = dev.upload_mx(rkhip.FP4, rows, cols, w, s)
    try:
        want = oracle.matvec_fp4(w, s, x, rows, cols, bf16=False)
        assert np.isinf(want).any() and np.isnan(want).any()
        check_both(dev, m, x, lambda r: oracle.matvec_fp4(w, s, x, rows, cols, bf16=r))
    finally:
        m.free()


def test_fp8_sum_rounds_to_even(dev):
    """internal/gpu/mx_test.go:180-238."""
    cols = 32
    x = np.zeros(cols, np.float32)
    x[0] = x[1] = x[2] = 256
    x[3] = 2.0 ** -9
    rows = []
    for low in (0x81, 0x82):
        row = [int(oracle.encode_e4m3([0.5])[0]), 2, 1, low]
        rows.append(row)
        rows.append([b ^ 0x80 for b in row])
    rows.append([int(oracle.encode_e4m3([448])[0])] * cols)
    w = np.zeros((len(rows), cols), np.uint8)
    for i, r in enumerate(rows):
        w[i, :len(r)] = r
    w = w.ravel()
    s = np.array([127], np.uint8)
    xb = x.copy()
    xb[4:] = 448
    m = dev.upload_mx(rkhip.FP8, len(rows), cols, w, s)
    try:
        for inp in (x, xb):
            want = oracle.matvec_fp8(w, s, inp, len(rows), cols)
            if inp[4] == 0:
                assert list(want[:4]) == [130, -130, 130, -130]
            same_bits(dev.matvecs([m], inp)[0], want, "rounds to even")
    finally:
        m.free()


def test_fp8_tie_stays_even_and_cancellation(dev):
    """internal/gpu/mx_test.go:240-267 and 298-328."""
    cols = 64
    x = np.zeros(cols, np.float32)
    x[0], x[1], x[32] = 256, 2.0 ** -9, 256
    w = np.zeros(cols, np.uint8)
    w[0], w[1], w[32] = oracle.encode_e4m3([0.5])[0], 2, 1
    s = np.array([127, 127], np.uint8)
    m = dev.upload_mx(rkhip.FP8, 1, cols, w, s)
    try:
        assert dev.matvecs([m], x)[0][0] == 128
    finally:
        m.free()
    cols = 32
    x = np.zeros(cols, np.float32)
    w = np.zeros(cols, np.uint8)
    x[0] = 448
    for i in range(1, 32):
        x[i], w[i] = 256, oracle.encode_e4m3([3.5])[0]
        if i > 16:
            w[i] |= 0x80
    x[16], w[16] = 0.9375, oracle.encode_e4m3([15.0 / 512])[0]
    m = dev.upload_mx(rkhip.FP8, 1, cols, w, np.array([127], np.uint8))
    try:
        m.set_raw(True)
        assert dev.matvecs([m], x)[0][0] == np.float32(225 * 2.0 ** -13)
    finally:
        m.free()


def test_large_fp8_matrix(dev):
    """internal/gpu/mx_test.go:269-296: 33000 x 4096."""
    rng = np.random.default_rng(10)
    rows, cols = 33000, 4096
    w, s = random_fp8(rng, rows, cols)
    x = mx_input(rng, cols)
    m = dev.upload_mx(rkhip.FP8, rows, cols, w, s)
    try:
        check_both(dev, m, x, lambda r: oracle.matvec_fp8(w, s, x, rows, cols, bf16=r))
    finally:
        m.free()


def test_quantize_fp8_and_batch_products(dev):
    """internal/gpu/mx_test.go:98-127 QuantizeFP8 through an arena (codes and
    scales as num.QuantizeActFP8), and MatVecs of FP8 and FP4 matrices with
    a float32 one in one batch (batch.go:214-264)."""
    rng = np.random.default_rng(6)
    cols = 4096
    x = mx_input(rng, cols, specials=True)
    want_c, want_s = oracle.act_fp8(x)
    w8, s8 = random_fp8(rng, 96, cols)
    w4 = rng.integers(0, 256, 80 * cols // 2).astype(np.uint8)
    s4 = random_scales(rng, 80 * cols // 32)
    wf = rng.normal(0, 1, 16 * cols).astype(np.float32)
    ms = [dev.upload_mx(rkhip.FP8, 96, cols, w8, s8), dev.upload_mx(rkhip.FP4, 80, cols, w4, s4),
          dev.upload(rkhip.F32, 16, cols, wf)]
    qx, xs = cols + 192, cols + 192 + cols  # E4M3 values take cols words
    arena = dev.arena(xs + cols // 32, 3 * cols)
    arena.set_quant_scratch(qx, xs)
    try:
        b = arena.begin()
        b.write(0, x)
        assert b.quantize_fp8(0, cols) == 0
        vals = b.read(qx, cols)
        scales = b.read(xs, cols // 32)
        b.submit()
        same_values(np.asarray(vals), e4m3_f32(want_c), "QuantizeFP8 values")
        assert np.array_equal(bits(scales), bits(want_s))
        b = arena.begin()
        b.write(0, x)
        b.matvecs(ms, [cols, cols + 96, cols + 176], 0)
        got = b.read(cols, 192)
        b.submit()
        got = np.asarray(got)
        same_bits(got[:96], oracle.matvec_fp8(w8, s8, x, 96, cols), "batch fp8")
        same_bits(got[96:176], oracle.matvec_fp4(w4, s4, x, 80, cols), "batch fp4")
        same_bits(got[176:], oracle.matvec32(wf, x, 16, cols), "batch f32")
    finally:
        arena.free()
        for m in ms:
            m.free()
    assert dev.used == 0


def test_mx_errors(dev):
    """device.go:626-640 and batch.go:221-238: NaN E4M3 weights, a width not
    a multiple of 32, Q8_0 and FP8 products of one input, and no batched
    prefill kernel for these formats."""
    with pytest.raises(rkhip.RKError, match="NaN in E4M3 weights") as e:
        dev.upload_mx(rkhip.FP8, 1, 32, np.full(32, 0x7F, np.uint8), np.array([127], np.uint8))
    assert e.value.code == -1
    with pytest.raises(rkhip.RKError, match="wrong shape"):
        dev.upload_mx(rkhip.FP4, 1, 48, np.zeros(24, np.uint8), np.zeros(2, np.uint8))
    q, s = oracle.quantize8(np.ones(64, np.float32))
    m8 = dev.upload_mx(rkhip.FP8, 2, 32, np.zeros(64, np.uint8), np.array([127], np.uint8))
    mq = dev.upload_q8(q, s, 2, 32)
    try:
        with pytest.raises(rkhip.RKError, match="Q8_0 and FP8 products of one input"):
            dev.matvecs([mq, m8], np.ones(32, np.float32))
        with pytest.raises(rkhip.RKError) as e:
            dev.matmul_t([m8], np.ones((2, 32), np.float32))
        assert e.value.code == -4
    finally:
        m8.free()
        mq.free()
    assert dev.used == 0


def test_batch_input_at_any_word(dev):
    """Products of an input at arena words 3 and 4 (unaligned and aligned
    to 16 bytes): the CPU's bits either way."""
    rng = np.random.default_rng(8)
    cols, r8, r4 = 2304, 70, 50
    x = mx_input(rng, cols, specials=True)
    w8, s8 = random_fp8(rng, r8, cols)
    w4 = rng.integers(0, 256, r4 * cols // 2).astype(np.uint8)
    s4 = random_scales(rng, r4 * cols // 32)
    ms = [dev.upload_mx(rkhip.FP8, r8, cols, w8, s8), dev.upload_mx(rkhip.FP4, r4, cols, w4, s4)]
    base = cols + 8
    arena = dev.arena(base + r8 + r4 + cols, 2 * cols)
    arena.set_quant_scratch(base + r8 + r4, base + r8 + r4 + cols // 4)
    try:
        for off in (3, 4):
            b = arena.begin()
            b.write(off, x)
            b.matvecs(ms, [base, base + r8], off)
            got = np.asarray(b.read(base, r8 + r4))
            b.submit()
            same_bits(got[:r8], oracle.matvec_fp8(w8, s8, x, r8, cols), f"fp8, input at word {off}")
            same_bits(got[r8:], oracle.matvec_fp4(w4, s4, x, r4, cols), f"fp4, input at word {off}")
    finally:
        arena.free()
        for m in ms:
            m.free()
    assert dev.used == 0


@pytest.mark.parametrize("cols,div", [(2304, 0), (2304, 1), (5120, 2)])
def test_expert_matvecs(dev, cols, div):
    """internal/gpu/dsbatch.go:142-172 ExpertMatVecs: selected E2M1 experts
    (ids in arena words, repeats allowed, an id past the last expert
    skipped) times inputs shared by all slots (div 0), one a slot (div 1) or
    one per two slots, each slot's output the CPU's product of its expert
    and input; the skipped slot's output is left as it was."""
    rng = np.random.default_rng(cols + div)
    E, P = 5, 40
    ids = np.array([3, 0, 3, 7, 1, 4], np.uint32)
    slots = ids.size
    w = rng.integers(0, 256, E * P * cols // 2).astype(np.uint8)
    s = random_scales(rng, E * P * cols // 32)
    d = slots if div == 0 else div
    inputs = (slots + d - 1) // d
    xs = [mx_input(rng, cols, specials=True) for _ in range(inputs)]
    m = dev.upload_mx(rkhip.FP4, E * P, cols, w, s)
    in0, idw, out0 = 0, inputs * cols, inputs * cols + 8
    words = out0 + slots * P + 64
    arena = dev.arena(words + cols, 2 * words)
    arena.set_quant_scratch(words, words + cols // 4)
    try:
        b = arena.begin()
        for k, x in enumerate(xs):
            b.write(in0 + k * cols, x)
        b.write(idw, ids.view(np.float32))
        b.write(out0, np.full(slots * P, 7.0, np.float32))
        assert b.expert_matvecs(m, P, idw, slots, in0, cols, div, out0, P) == 0
        got = np.asarray(b.read(out0, slots * P)).reshape(slots, P)
        b.submit()
        for k, e in enumerate(ids):
            if e >= E:
                assert np.all(got[k] == 7.0), "skipped slot written"
                continue
            want = oracle.matvec_fp4(w[e * P * cols // 2:(e + 1) * P * cols // 2], s[e * P * cols // 32:(e + 1) * P * cols // 32],
                                     xs[k // d], P, cols)
            same_bits(got[k], want, f"slot {k} expert {e}")
    finally:
        arena.free()
        m.free()
    assert dev.used == 0


@pytest.mark.parametrize("rows,cols", [(7, 32), (300, 896), (1000, 1280), (40, 5120), (33, 9216)])
def test_matvecs_batch(dev, rows, cols):
    """internal/gpu/mx_test.go:371-420 MatVecsBatch: an E4M3 matrix times
    1, 3, 8, 11 and 17 inputs, rounded and raw, each output the CPU's
    product."""
    rng = np.random.default_rng(rows + cols)
    w, s = random_fp8(rng, rows, cols)
    m = dev.upload_mx(rkhip.FP8, rows, cols, w, s)
    nmax = 17
    words = nmax * cols + nmax * rows + 64
    arena = dev.arena(words + cols, nmax * (cols + rows) + 64)
    arena.set_quant_scratch(words, words + cols // 4)
    try:
        for raw in (False, True):
            m.set_raw(raw)
            for n in (1, 3, 8, 11, 17):
                xs = [mx_input(rng, cols) for _ in range(n)]
                b = arena.begin()
                for j in range(n):
                    b.write(j * cols, xs[j])
                out = n * cols
                assert b.matvecs_batch(m, out, rows, 0, cols, n) == 0
                got = np.asarray(b.read(out, n * rows)).reshape(n, rows)
                b.submit()
                for j in range(n):
                    same_bits(got[j], oracle.matvec_fp8(w, s, xs[j], rows, cols, bf16=not raw),
                              f"{rows}x{cols} input {j} of {n} raw {raw}")
    finally:
        arena.free()
        m.free()
    assert dev.used == 0


def test_in_place_quantizers(dev):
    """internal/gpu/dsbatch.go:60-74 ActQuantInPlace and FP4QuantInPlace
    (both scale kinds) against the oracle, which equals the reference
    kernels' act_quant / fp4_act_quant vectors (test_oracle_mx.py): the
    reference's own inputs, then random blocks (zero, huge, tiny, ties,
    denormals, signed zeros), then blocks holding an infinity or a NaN.
    Those make NaNs (0·inf, 0/-0): they must sit at the oracle's positions
    and every other value must match bit for bit, but a NaN's sign is not
    pinned (the CPU path's x86 multiply gives the negative default NaN, the
    GPU a positive one), so NaNs match any NaN."""
    with gzip.open(GOLDEN, "rt") as f:
        vec = json.load(f)
    rng = np.random.default_rng(13)
    cases = [bf16s(c["x"]) for c in vec["act_quant"]] + [mx_input(rng, 4096), mx_input(rng, 96),
                                                        mx_input(rng, 4096, specials=True)]
    fcases = [bf16s(c["x"]) for c in vec["fp4_quant"]] + [mx_input(rng, 4096), mx_input(rng, 64),
                                                         mx_input(rng, 4096, specials=True)]
    arena = dev.arena(8192, 16384)
    try:
        for x in cases:
            b = arena.begin()
            b.write(0, x)
            assert b.act_quant_inplace(0, x.size) == 0
            got = np.asarray(b.read(0, x.size))
            b.submit()
            same_values(got, oracle.act_quant_inplace(x), f"act quant of {x.size}")
        for x in fcases:
            for e4m3 in (False, True):
                b = arena.begin()
                b.write(0, x)
                assert b.fp4_quant_inplace(0, x.size, e4m3) == 0
                got = np.asarray(b.read(0, x.size))
                b.submit()
                p_, s_ = oracle.quantize_fp4(x, e4m3)
                same_values(got, oracle.dequant_fp4(p_, s_, x.size, e4m3), f"fp4 quant of {x.size} e4m3={e4m3}")
    finally:
        arena.free()


def test_words_past_the_quantized_input_read_from_the_arena(dev):
    """internal/gpu/mx_test.go:98-127: after QuantizeFP8 of n floats, n words
    at qxOff hold the E4M3 values, unscaled, and n/32 at xsOff the scales;
    words beyond them are the arena's own. A product afterwards leaves those
    words as they were."""
    rng = np.random.default_rng(21)
    cols = 256
    x = mx_input(rng, cols)
    qx, xs = 1024, 1024 + cols
    arena = dev.arena(4096, 8192)
    arena.set_quant_scratch(qx, xs)
    w8, s8 = random_fp8(rng, 40, cols)
    m = dev.upload_mx(rkhip.FP8, 40, cols, w8, s8)
    try:
        b = arena.begin()
        b.write(0, x)
        b.write(xs + cols // 32, np.arange(64, dtype=np.float32))  # after the scales
        assert b.quantize_fp8(0, cols) == 0
        vals = np.asarray(b.read(qx, cols))
        scales = np.asarray(b.read(xs, cols // 32))
        after = np.asarray(b.read(xs + cols // 32, 64))
        b.submit()
        want_c, want_s = oracle.act_fp8(x)
        same_values(vals, e4m3_f32(want_c), "QuantizeFP8 values")
        assert np.array_equal(bits(scales), bits(want_s))
        assert np.array_equal(after, np.arange(64, dtype=np.float32))
        # a product of another input: the reserved words keep the values
        b = arena.begin()
        b.write(0, -x)
        b.matvecs([m], [2048], 0)
        again = np.asarray(b.read(qx, cols))
        got = np.asarray(b.read(2048, 40))
        b.submit()
        same_values(again, vals, "reserved words after a product")
        same_bits(got, oracle.matvec_fp8(w8, s8, -x, 40, cols), "product after QuantizeFP8")
    finally:
        arena.free()
        m.free()


def e4m3_f32(codes):
    """The E4M3 codes' values as float32 (NaN for the NaN codes)."""
    return oracle.e4m3_values()[np.asarray(codes)].astype(np.float32)


def same_values(got, want, what):
    """Bit-equal, except that a NaN matches any NaN (the NaN codes' values
    carry no pinned payload)."""
    g, w = np.asarray(got, np.float32), np.asarray(want, np.float32)
    nan = np.isnan(w)
    assert np.array_equal(np.isnan(g), nan), f"{what}: NaN positions differ"
    same_bits(g[~nan], w[~nan], what)


def test_chunked_stacked_experts(dev):
    """device.go:575-581, 609-618, 704-723: stacked experts given as pieces
    (Format{FP4Chunks, E8M0Chunks, AlignRows}, as dsv41/gpu.go:177-184 makes
    them, one piece an expert) equal the matrix uploaded whole, bit for bit,
    and the oracle; pieces cut anywhere (not at rows) read as one; E4M3
    scales in pieces too."""
    rng = np.random.default_rng(44)
    experts, erows, cols = 6, 96, 512
    rows = experts * erows
    x = mx_input(rng, cols)
    ws = [rng.integers(0, 256, erows * cols // 2).astype(np.uint8) for _ in range(experts)]
    ss = [random_scales(rng, erows * cols // 32) for _ in range(experts)]
    w, s = np.concatenate(ws), np.concatenate(ss)
    whole = dev.upload_mx(rkhip.FP4, rows, cols, w, s)
    per_expert = dev.upload_mx_chunks(rkhip.FP4, rows, cols, ws, ss, align_rows=erows)
    cut = [0, 1, 1000, 1001, 77777, w.size]
    odd = dev.upload_mx_chunks(rkhip.FP4, rows, cols, [w[a:b] for a, b in zip(cut, cut[1:])],
                               [s[:5], s[5:5], s[5:]])
    try:
        want = oracle.matvec_fp4(w, s, x, rows, cols, bf16=True)
        for m in (whole, per_expert, odd):
            same_bits(dev.matvec(m, x), want, "chunked FP4")
        fw, fs = random_fp8(rng, 64, 256)
        m8 = dev.upload_mx_chunks(rkhip.FP8, 64, 256, [fw[:3000], fw[3000:]], [fs[:7], fs[7:]], align_rows=32)
        try:
            same_bits(dev.matvec(m8, x[:256]), oracle.matvec_fp8(fw, fs, x[:256], 64, 256, bf16=True), "chunked FP8")
        finally:
            m8.free()
    finally:
        for m in (whole, per_expert, odd):
            m.free()
    assert dev.used == 0


def test_chunked_upload_errors(dev):
    """The reference's checks on pieces (device.go:604-618): the pieces'
    total against the shape, the scales' count, NaN codes in any piece, and
    AlignRows (whole runs; E4M3 runs of a multiple of 32 rows)."""
    z = lambda n: np.zeros(n, np.uint8)  # noqa: E731
    with pytest.raises(rkhip.RKError, match="out of range"):
        dev.upload_mx_chunks(rkhip.FP4, 4, 64, [z(64), z(63)], [z(8)])
    with pytest.raises(rkhip.RKError, match="wrong shape"):
        dev.upload_mx_chunks(rkhip.FP4, 4, 64, [z(64), z(64)], [z(7)])
    with pytest.raises(rkhip.RKError, match="NaN in E4M3 weights"):
        dev.upload_mx_chunks(rkhip.FP8, 2, 32, [z(40), np.full(24, 0xFF, np.uint8)], [np.array([127], np.uint8)])
    with pytest.raises(rkhip.RKError, match="aligned runs"):
        dev.upload_mx_chunks(rkhip.FP4, 6, 64, [z(192)], [z(12)], align_rows=4)
    with pytest.raises(rkhip.RKError, match="aligned runs"):
        dev.upload_mx_chunks(rkhip.FP8, 64, 32, [z(2048)], [z(2)], align_rows=16)
    m = dev.upload_mx_chunks(rkhip.FP4, 6, 64, [z(192)], [z(12)], align_rows=3)
    m.free()
    assert dev.used == 0
