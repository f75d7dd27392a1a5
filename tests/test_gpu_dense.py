"""float32 and bfloat16 products on the GPU (internal/num/matvec.go:106-123
MatVec32 / MatVecBF16 through internal/gpu Upload + MulVecs), bit for bit
against the CPU oracle: odd widths (the padded tail), widths past the
input's LDS staging, rows past a wave's eight, special values, mixed
formats in one call, the batch path without a quantize scratch, and the
reference's shape errors."""
import numpy as np
import pytest

import rkhip
from oracle import oracle

pytestmark = pytest.mark.gpu


def same_bits(got, want, what):
    g, w = np.ascontiguousarray(got).view(np.uint32), np.ascontiguousarray(want).view(np.uint32)
    if not np.array_equal(g, w):
        i = int(np.argmax(g != w))
        raise AssertionError(f"{what}: row {i}: GPU {got[i]!r} ({g[i]:#x}), oracle {want[i]!r} ({w[i]:#x}), "
                             f"{int(np.sum(g != w))} rows differ")


def awkward(rng, n, scale=1.0):
    """Normal values plus denormals, -0, infinities and NaNs (rarely)."""
    v = (rng.normal(0, 1, n) * scale).astype(np.float32)
    pick = rng.integers(0, 60, n)
    den = rng.integers(0, 1 << 23, n, dtype=np.uint32).view(np.float32)
    v[pick == 0] = den[pick == 0]
    v[pick == 1] = np.float32(-0.0)
    v[pick == 2] = np.float32(1e-30)
    return v


def to_bf16(v):
    """Round to nearest even bfloat16 (numpy restatement of
    internal/num/matvec.go:22-29 ToBF16, for building inputs)."""
    b = v.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = v != v
    r[nan] = ((b[nan] >> 16).astype(np.uint16)) | 0x40
    return r


SHAPES = [(1, 1), (3, 7), (8, 32), (9, 33), (300, 896), (67, 4865), (1024, 4096), (5, 40001)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_f32_matvec_matches_cpu(dev, rows, cols):
    rng = np.random.default_rng(rows * 7919 + cols)
    w = awkward(rng, rows * cols)
    x = awkward(rng, cols)
    m = dev.upload(rkhip.F32, rows, cols, w)
    try:
        same_bits(dev.matvec(m, x), oracle.matvec32(w, x, rows, cols), f"f32 {rows}x{cols}")
    finally:
        m.free()
    assert dev.used == 0


@pytest.mark.parametrize("rows,cols", [s for s in SHAPES if s[1] % 2 == 0] + [(33, 2), (129, 18944)])
def test_bf16_matvec_matches_cpu(dev, rows, cols):
    rng = np.random.default_rng(rows * 31 + cols)
    w16 = to_bf16(awkward(rng, rows * cols))
    x = awkward(rng, cols)
    m = dev.upload(rkhip.BF16, rows, cols, w16)
    try:
        same_bits(dev.matvec(m, x), oracle.matvec_bf16(w16, x, rows, cols), f"bf16 {rows}x{cols}")
    finally:
        m.free()
    assert dev.used == 0


def test_specials_propagate_like_cpu(dev):
    """Infinities and NaNs in weights and input: each row's bits are the
    oracle's (canonical handling is the reference's: none in MatVec32)."""
    rng = np.random.default_rng(3)
    rows, cols = 64, 256
    w = rng.normal(0, 1, rows * cols).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    w[5 * cols + 3] = np.inf
    w[9 * cols + 100] = -np.inf
    w[17 * cols + 7] = np.nan
    w[20 * cols + 1] = np.inf
    w[20 * cols + 33] = -np.inf  # inf - inf in one running sum
    x[200] = np.float32(3e38)
    w[40 * cols + 200] = np.float32(3e38)  # overflow to inf
    for kind, ww, ref in ((rkhip.F32, w, oracle.matvec32(w, x, rows, cols)),):
        m = dev.upload(kind, rows, cols, ww)
        try:
            same_bits(dev.matvec(m, x), ref, "specials")
        finally:
            m.free()


def test_mixed_formats_one_call(dev):
    """One MulVecs over Q8, float32 and bfloat16 matrices of one input
    (internal/gpu/device.go:769-793): each output is its format's CPU
    product."""
    rng = np.random.default_rng(9)
    cols = 512
    x = rng.normal(0, 1, cols).astype(np.float32)
    wf = rng.normal(0, 0.1, 100 * cols).astype(np.float32)
    wb = to_bf16(rng.normal(0, 0.1, 70 * cols).astype(np.float32))
    q, s = oracle.quantize8(rng.normal(0, 0.1, 50 * cols).astype(np.float32))
    ms = [dev.upload(rkhip.F32, 100, cols, wf), dev.upload_q8(q, s, 50, cols), dev.upload(rkhip.BF16, 70, cols, wb)]
    try:
        outs = dev.matvecs(ms, x)
        same_bits(outs[0], oracle.matvec32(wf, x, 100, cols), "f32 of three")
        same_bits(outs[1], oracle.matvec_q8(q, s, x, 50, cols), "q8 of three")
        same_bits(outs[2], oracle.matvec_bf16(wb, x, 70, cols), "bf16 of three")
    finally:
        for m in ms:
            m.free()
    assert dev.used == 0


def test_batch_dense_products_need_no_quant_scratch(dev):
    """internal/gpu/batch.go:214-264: a float product reads the input as it
    is, so an arena without a quantize scratch runs it."""
    rng = np.random.default_rng(12)
    rows, cols = 96, 320
    w = rng.normal(0, 1, rows * cols).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    m = dev.upload(rkhip.F32, rows, cols, w)
    arena = dev.arena(cols + rows, cols + rows)
    try:
        b = arena.begin()
        b.write(0, x)
        b.matvecs([m], [cols], 0)
        got = b.read(cols, rows)
        b.submit()
        same_bits(np.asarray(got), oracle.matvec32(w, x, rows, cols), "batch f32")
    finally:
        arena.free()
        m.free()
    assert dev.used == 0


def test_dense_shape_errors(dev):
    """internal/gpu/device.go:593-595: bfloat16 rows need an even width;
    the batched prefill has no float kernel in this build."""
    with pytest.raises(rkhip.RKError) as e:
        dev.upload(rkhip.BF16, 4, 7, np.zeros(28, np.uint16))
    assert e.value.code == -1
    m = dev.upload(rkhip.F32, 4, 32, np.zeros(128, np.float32))
    try:
        with pytest.raises(rkhip.RKError) as e:
            dev.matmul_t([m], np.zeros((2, 32), np.float32))
        assert e.value.code == -4
    finally:
        m.free()
    assert dev.used == 0
