"""Q8_0 / Q4_0 products on the GPU, bit for bit against the CPU oracle
(the reference's TestKernelsMatchCPUBitForBit, internal/gpu/gpu_test.go:59-141,
plus the benchmark shapes)."""
import numpy as np
import pytest

import rkhip
from oracle import oracle

pytestmark = pytest.mark.gpu


def awkward(rng, n, scale):
    """internal/gpu/gpu_test.go:35-48: normal values plus denormals, -0 and
    1e-30, each with probability 1/40."""
    v = (rng.normal(0, 1, n) * scale).astype(np.float32)
    pick = rng.integers(0, 40, n)
    den = rng.integers(0, 1 << 23, n, dtype=np.uint32).view(np.float32)
    v[pick == 0] = den[pick == 0]
    v[pick == 1] = np.float32(-0.0)
    v[pick == 2] = np.float32(1e-30)
    return v


def same_bits(got, want, what):
    g, w = got.view(np.uint32), want.view(np.uint32)
    if not np.array_equal(g, w):
        i = int(np.argmax(g != w))
        raise AssertionError(f"{what}: row {i}: GPU {got[i]!r} ({g[i]:#x}), oracle {want[i]!r} ({w[i]:#x}), "
                             f"{int(np.sum(g != w))} rows differ")


@pytest.mark.parametrize("rows,cols", [(7, 32), (300, 896), (64, 4864), (1000, 96), (33, 288), (5, 768)])
def test_awkward_inputs_match(dev, rows, cols):
    rng = np.random.default_rng(rows * 7919 + cols)
    w = awkward(rng, rows * cols, 0.05)
    x = awkward(rng, cols, 1.0)
    q8, s8 = oracle.quantize8(w)
    m = dev.upload_q8(q8, s8, rows, cols)
    same_bits(dev.matvec(m, x), oracle.matvec_q8(q8, s8, x, rows, cols), f"q8 {rows}x{cols}")
    m.free()
    q4, s4 = oracle.quantize4(w)
    m = dev.upload_q4(q4, s4, rows, cols)
    same_bits(dev.matvec(m, x), oracle.matvec_q4(q4, s4, x, rows, cols), f"q4 {rows}x{cols}")
    m.free()
    assert dev.used == 0


@pytest.mark.parametrize("rows,cols", [(300000, 32), (40000, 1024)])
def test_large_matrices(dev, rows, cols):
    rng = np.random.default_rng(rows)
    q = rng.integers(-127, 128, rows * cols, dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, rows * cols // 32).astype(np.float32)
    x = awkward(rng, cols, 1.0)
    m = dev.upload_q8(q, s, rows, cols)
    same_bits(dev.matvec(m, x), oracle.matvec_q8(q, s, x, rows, cols), f"q8 {rows}x{cols}")
    m.free()


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_benchmark_shapes_q8(dev, rows, cols):
    """Config 2: codes uniform in [-127, 127], scales U(1e-3, 1e-2), x N(0,1)."""
    rng = np.random.default_rng(cols * 3 + rows)
    q = rng.integers(-127, 128, rows * cols, dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, rows * cols // 32).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    m = dev.upload_q8(q, s, rows, cols)
    same_bits(dev.matvec(m, x), oracle.matvec_q8(q, s, x, rows, cols), f"q8 {rows}x{cols}")
    m.free()


@pytest.mark.parametrize("rows,cols", [(512, 3584), (512, 18944), (1000, 2048), (64, 14336)])
def test_q4_shapes(dev, rows, cols):
    """Config 4's widths (3584 = 112 blocks, 18944 = 592: partial chunks)."""
    rng = np.random.default_rng(cols + rows)
    q = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    s = rng.uniform(1e-3, 1e-2, rows * cols // 32).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    m = dev.upload_q4(q, s, rows, cols)
    same_bits(dev.matvec(m, x), oracle.matvec_q4(q, s, x, rows, cols), f"q4 {rows}x{cols}")
    m.free()


def test_several_matrices_one_input(dev):
    """MulVecs of Q/K/V-like matrices, mixed Q8/Q4 (q4_m keeps V in Q8), and
    more matrices than one launch takes."""
    rng = np.random.default_rng(21)
    cols = 896
    shapes = [(896, "q8"), (128, "q4"), (128, "q8"), (4864, "q4"), (4864, "q8"), (7, "q8"), (33, "q4")]
    x = awkward(rng, cols, 1.0)
    ms, wants = [], []
    for rows, kind in shapes:
        w = rng.normal(0, 0.05, rows * cols).astype(np.float32)
        if kind == "q8":
            q, s = oracle.quantize8(w)
            ms.append(dev.upload_q8(q, s, rows, cols))
            wants.append(oracle.matvec_q8(q, s, x, rows, cols))
        else:
            q, s = oracle.quantize4(w)
            ms.append(dev.upload_q4(q, s, rows, cols))
            wants.append(oracle.matvec_q4(q, s, x, rows, cols))
    for i, (got, want) in enumerate(zip(dev.matvecs(ms, x), wants)):
        same_bits(got, want, f"matrix {i}")
    for m in ms:
        m.free()
    assert dev.used == 0


def test_zero_and_tiny_inputs(dev):
    """All-zero input (scale 0, codes 0), a block of only denormals (its
    reciprocal scale overflows), and blocks of -0."""
    rng = np.random.default_rng(22)
    rows, cols = 64, 256
    q = rng.integers(-127, 128, rows * cols, dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, rows * cols // 32).astype(np.float32)
    m = dev.upload_q8(q, s, rows, cols)
    xs = [np.zeros(cols, np.float32), np.full(cols, -0.0, np.float32)]
    x = rng.normal(0, 1, cols).astype(np.float32)
    x[:32] = rng.integers(1, 1 << 20, 32, dtype=np.uint32).view(np.float32)
    x[32:64] = 0
    x[40] = np.float32(1e-44)
    xs.append(x)
    for x in xs:
        same_bits(dev.matvec(m, x), oracle.matvec_q8(q, s, x, rows, cols), "q8 special input")
    m.free()


@pytest.mark.parametrize("n", [32, 288, 4096])
def test_batch_quantize_leaves_codes_in_the_arena(dev, n):
    """internal/gpu/batch.go:277-280 Quantize through an arena: the Q8_0
    codes four a word (code j in byte j, kernels.go:340-349) at qxOff and
    the block scales at xsOff, as num.QuantizeActs gives them; the word
    after the scales is the arena's own, and a product afterwards (which
    quantizes into its own scratch) leaves the reserved words as they were."""
    rng = np.random.default_rng(n)
    x = awkward(rng, n, 1.0)
    x[:32] = 0.0  # an all-zero block: scale 0, codes 0
    want_q, want_s = oracle.quantize8(x)
    qx, xs = 2 * n, 2 * n + n // 4
    arena = dev.arena(xs + n // 32 + 1 + 64, 4 * n + 64)
    arena.set_quant_scratch(qx, xs)
    rows = 64
    q8, s8 = oracle.quantize8(rng.normal(0, 0.05, rows * n).astype(np.float32))
    m = dev.upload_q8(q8, s8, rows, n)
    try:
        b = arena.begin()
        b.write(0, x)
        b.write(xs + n // 32, np.array([1.5], np.float32))
        assert b.quantize(0, n) == 0
        codes = b.read(qx, n // 4)
        scales = b.read(xs, n // 32)
        after = b.read(xs + n // 32, 1)
        b.submit()
        assert np.array_equal(np.asarray(codes).view(np.int8), want_q)
        same_bits(np.asarray(scales), want_s, "Quantize scales")
        assert after[0] == 1.5
        b = arena.begin()
        b.write(n, -x)
        b.matvecs([m], [xs + n // 32 + 1], n)
        again = b.read(qx, n // 4)
        got = b.read(xs + n // 32 + 1, rows)
        b.submit()
        assert np.array_equal(np.asarray(again).view(np.int8), want_q)
        same_bits(np.asarray(got), oracle.matvec_q8(q8, s8, -x, rows, n), "product after Quantize")
    finally:
        arena.free()
        m.free()
    assert dev.used == 0


def test_shape_errors(dev):
    rng = np.random.default_rng(23)
    q = rng.integers(-127, 128, 64 * 64, dtype=np.int8)
    s = np.ones(64 * 2, np.float32)
    with pytest.raises(rkhip.RKError) as e:
        dev.upload_q8(q, s, 64, 48)  # cols not a multiple of 32
    assert e.value.code == rkhip.RK_ERR_ARGS
    m = dev.upload_q8(q, s, 64, 64)
    with pytest.raises(rkhip.RKError) as e:
        dev.matvecs([m], np.zeros(32, np.float32))
    assert e.value.code == rkhip.RK_ERR_ARGS
    m.free()
    assert dev.used == 0


def test_out_of_memory_is_an_error_and_the_device_stays_usable(dev):
    """The failure internal/llm/model.go:168-188 falls back from: a request
    for more device memory than the GPU has (an arena of 400 GB on a 288 GB
    MI355X; hipMalloc refuses it before anything else happens) returns
    RK_ERR_OOM with its text, does not abort, leaves Used() as it was, and
    the next products on the device still give the CPU's bits, as does a
    product call that fails (a submission of more rows than one call takes)."""
    rng = np.random.default_rng(26)
    rows, cols = 512, 4096
    q = rng.integers(-127, 128, rows * cols, dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, rows * cols // 32).astype(np.float32)
    m = dev.upload_q8(q, s, rows, cols)
    used = dev.used
    x = rng.normal(0, 1, cols).astype(np.float32)
    with pytest.raises(rkhip.RKError) as e:
        dev.arena(100_000_000_000, 16)  # 400 GB of words
    assert e.value.code == rkhip.RK_ERR_OOM
    assert "arena" in str(e.value) and "memory" in str(e.value).lower(), str(e.value)
    assert dev.used == used
    same_bits(dev.matvec(m, x), oracle.matvec_q8(q, s, x, rows, cols), "product after the failed allocation")
    with pytest.raises(rkhip.RKError) as e:
        dev.matvecs([m] * 2049, x)  # 2049 · 512 rows > 2^20 in one submission
    assert e.value.code == rkhip.RK_ERR_ARGS
    same_bits(dev.matvec(m, x), oracle.matvec_q8(q, s, x, rows, cols), "product after the failed call")
    m.free()
    assert dev.used == 0


def test_device_pointers(dev):
    """rk_matvecs_device on device addresses inside an arena (the stream:
    the device's own), then read back through a batch."""
    rng = np.random.default_rng(24)
    rows, cols = 2048, 4096
    q = rng.integers(-127, 128, rows * cols, dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, rows * cols // 32).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    m = dev.upload_q8(q, s, rows, cols)
    a = dev.arena(cols + rows, cols + rows)
    b = a.begin()
    b.write(0, x)
    b.submit()
    dev.matvecs_device([m], [a.device_ptr(cols)], a.device_ptr(0), cols)
    b = a.begin()
    out = b.read(cols, rows)
    b.submit()
    same_bits(out, oracle.matvec_q8(q, s, x, rows, cols), "device-pointer q8")
    a.free()
    m.free()
    assert dev.used == 0


def test_graph_replays_match(dev):
    """Products recorded once into a graph and replayed: each replay reads
    the arena's current input (changed by eager batches between replays)
    and gives the oracle's bits for it."""
    rng = np.random.default_rng(25)
    cols = 2048
    q8 = rng.integers(-127, 128, 1000 * cols, dtype=np.int8)
    s8 = rng.uniform(1e-3, 1e-2, 1000 * cols // 32).astype(np.float32)
    q4 = rng.integers(0, 256, 300 * cols // 2, dtype=np.uint8)
    s4 = rng.uniform(1e-3, 1e-2, 300 * cols // 32).astype(np.float32)
    m8, m4 = dev.upload_q8(q8, s8, 1000, cols), dev.upload_q4(q4, s4, 300, cols)
    a = dev.arena(cols + 1300, cols + 1300)
    dev.graph_begin()
    dev.matvecs_device([m8, m4], [a.device_ptr(cols), a.device_ptr(cols + 1000)], a.device_ptr(0), cols)
    g = dev.graph_end()
    for rep in range(4):
        x = rng.normal(0, 1, cols).astype(np.float32)
        b = a.begin()
        b.write(0, x)
        b.write(cols, np.full(1300, np.nan, np.float32))  # stale outputs would show
        b.submit()
        g.launch(1)
        b = a.begin()
        o8, o4 = b.read(cols, 1000), b.read(cols + 1000, 300)
        b.submit()
        same_bits(o8, oracle.matvec_q8(q8, s8, x, 1000, cols), f"replay {rep} q8")
        same_bits(o4, oracle.matvec_q4(q4, s4, x, 300, cols), f"replay {rep} q4")
    g.free()
    a.free()
    m8.free()
    m4.free()
    assert dev.used == 0


def test_launch_floor(dev):
    """rk_device_launch_floor: an empty launch costs time, a plain read of
    18.9 MB costs more, and the read rate it implies stays under the HBM
    peak (the copies rotate past the MALL); bad arguments are errors."""
    nbytes = 18907136  # config 2's 4096x4096 product: codes, scales, input and output
    empty_us, read_us = dev.launch_floor(nbytes, copies=32, launches=50)
    assert 0.0 < empty_us < read_us
    assert nbytes / (read_us * 1e-6) < 8.0e12 * 1.05
    for args in [(0, 1, 1), (17, 1, 1), (nbytes, 0, 1), (nbytes, 1, 0)]:
        with pytest.raises(rkhip.RKError) as e:
            dev.launch_floor(*args)
        assert e.value.code == rkhip.RK_ERR_ARGS
