"""The oracle's rakkan_tensor_v1 operators (internal/sandbox/tensor.go)
pinned to the reference's known answers (internal/sandbox/tensor_test.go)
and to independent computations: numpy's int64 products for the exact i8
sums (wrapped to int32 as Go does), and a float32 scalar loop for the
sequential f32 sum."""
import numpy as np

from oracle import oracle


def test_int8_matmul_closed_form():
    """TestInt8MatmulIsExact (tensor_test.go:69-95): a.i8[i] = i%255-127
    (3x64), b.i8[i] = 127-i%200 (64x2)."""
    a = (np.arange(3 * 64) % 255 - 127).astype(np.int8).reshape(3, 64)
    b = (127 - np.arange(64 * 2) % 200).astype(np.int8).reshape(64, 2)
    want = a.astype(np.int64) @ b.astype(np.int64)
    got = oracle.tensor_matmul_i8(a, b, False)
    assert got.dtype == np.int32
    assert np.array_equal(got, want.astype(np.int32))
    assert np.array_equal(oracle.tensor_matmul_i8(a, np.ascontiguousarray(b.T), True), got)


def test_int8_matmul_wraps_like_go_int32():
    k = 140000  # 140000 * 127 * 127 > 2^31
    a = np.full((2, k), 127, np.int8)
    b = np.full((k, 3), 127, np.int8)
    b[:, 1] = -128
    want = (a.astype(np.int64) @ b.astype(np.int64)) & 0xFFFFFFFF
    want = np.where(want >= 1 << 31, want - (1 << 32), want).astype(np.int32)
    assert np.array_equal(oracle.tensor_matmul_i8(a, b, False), want)
    assert int(want[0, 0]) == 140000 * 16129 - (1 << 32)


def test_quantize_rounds_half_to_even_and_clamps():
    """TestQuantizeRoundsAndClamps (tensor_test.go:97-108)."""
    a = np.array([0.25, 0.75, -0.25, 1000, -1000], np.float32)
    assert list(oracle.tensor_quantize(a, 0.5)) == [0, 2, 0, 127, -127]


def test_quantize_matches_numpy_rint_of_the_f32_quotient():
    rng = np.random.default_rng(1)
    a = (rng.normal(0, 40, 100000)).astype(np.float32)
    a[:8] = [2.5, -2.5, 3.5, 126.5, 127.5, -127.5, np.inf, -np.inf]
    k = np.float32(0.37)
    q = np.rint(a / k)  # float32 quotient, round half to even
    want = np.clip(q, -127, 127).astype(np.int8)
    assert np.array_equal(oracle.tensor_quantize(a, k), want)


def test_scale_dequantizes():
    """TestSoftmaxAddReluScale's scale (tensor_test.go:138-142)."""
    assert list(oracle.tensor_scale_i32(np.array([4, -6], np.int32), 0.5)) == [2.0, -3.0]


def seq_matmul_f32(a, b):
    """A float32 scalar loop: acc += float32(a·b) in order, as refMatmul
    (tensor_test.go:26-38)."""
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n), np.float32)
    for i in range(m):
        for j in range(n):
            acc = np.float32(0)
            for p in range(k):
                acc = np.float32(acc + np.float32(a[i, p] * b[p, j]))
            out[i, j] = acc
    return out


def test_f32_matmul_is_the_sequential_sum_and_transposed_agrees():
    """TestMatmulExactAndTransposedAgrees (tensor_test.go:40-67): 7x33 by
    33x5 normal values."""
    rng = np.random.default_rng(2)
    a = rng.normal(0, 1, (7, 33)).astype(np.float32)
    b = rng.normal(0, 1, (33, 5)).astype(np.float32)
    c = oracle.tensor_matmul_f32(a, b, False)
    assert np.array_equal(c.view(np.uint32), seq_matmul_f32(a, b).view(np.uint32))
    ct = oracle.tensor_matmul_f32(a, np.ascontiguousarray(b.T), True)
    assert np.array_equal(c.view(np.uint32), ct.view(np.uint32))


def test_inf_times_zero_is_canonical_nan():
    """TestTensorNaNIsCanonical (tensor_test.go:145-153)."""
    c = oracle.tensor_matmul_f32(np.array([[np.inf]], np.float32), np.array([[0]], np.float32), False)
    assert int(c.view(np.uint32)[0, 0]) == 0x7FC00000
