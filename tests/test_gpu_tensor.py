"""rakkan_tensor_v1 matmul / matmul_t, quantize and scale on the GPU against
the oracle, bit for bit (internal/sandbox/tensor.go:286-339, 366-387,
445-461; the reference's cases in internal/sandbox/tensor_test.go)."""
import numpy as np
import pytest

import rkhip
from oracle import oracle
from test_gpu_matvec import awkward

pytestmark = pytest.mark.gpu


def bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


@pytest.mark.parametrize("m,k,n", [(7, 33, 5), (64, 64, 64), (100, 257, 70), (1, 4096, 1), (130, 1000, 33),
                                   (33, 3, 129)])
def test_f32_matmul_and_matmul_t(dev, m, k, n):
    rng = np.random.default_rng(m * 1000 + k + n)
    a = awkward(rng, m * k, 1.0).reshape(m, k)
    b = awkward(rng, k * n, 1.0).reshape(k, n)
    want = oracle.tensor_matmul_f32(a, b, False)
    assert np.array_equal(bits(dev.tensor_matmul(a, b)), bits(want))
    bt = np.ascontiguousarray(b.T)
    assert np.array_equal(bits(dev.tensor_matmul(a, bt, transposed=True)), bits(want))


def test_f32_inf_times_zero_is_canonical(dev):
    """TestTensorNaNIsCanonical: Inf·0 -> 0x7fc00000; and a NaN input with
    another payload comes out canonical too."""
    c = dev.tensor_matmul(np.array([[np.inf]], np.float32), np.array([[0]], np.float32))
    assert int(bits(c)[0, 0]) == 0x7FC00000
    odd = np.array([0x7FA00001], np.uint32).view(np.float32)
    c = dev.tensor_matmul(np.array([[1.0, odd[0]]], np.float32), np.array([[1.0], [1.0]], np.float32))
    assert int(bits(c)[0, 0]) == 0x7FC00000


def test_i8_closed_form(dev):
    """TestInt8MatmulIsExact (tensor_test.go:69-95)."""
    a = (np.arange(3 * 64) % 255 - 127).astype(np.int8).reshape(3, 64)
    b = (127 - np.arange(64 * 2) % 200).astype(np.int8).reshape(64, 2)
    c = dev.tensor_matmul(a, b)
    assert c.dtype == np.int32
    assert np.array_equal(c, oracle.tensor_matmul_i8(a, b, False))


@pytest.mark.parametrize("m,k,n", [(64, 256, 64), (70, 1000, 130), (1, 31, 1), (200, 3000, 17), (5, 70000, 9)])
def test_i8_matmul_and_matmul_t(dev, m, k, n):
    rng = np.random.default_rng(m + k * 3 + n * 7)
    a = rng.integers(-128, 128, (m, k), dtype=np.int16).astype(np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int16).astype(np.int8)
    want = oracle.tensor_matmul_i8(a, b, False)
    assert np.array_equal(dev.tensor_matmul(a, b), want)
    assert np.array_equal(dev.tensor_matmul(a, np.ascontiguousarray(b.T), transposed=True), want)


def test_i8_wraps_like_go_int32(dev):
    k = 140000
    a = np.full((2, k), 127, np.int8)
    b = np.full((k, 3), 127, np.int8)
    b[:, 1] = -128
    b[::7, 2] = -128
    assert np.array_equal(dev.tensor_matmul(a, b), oracle.tensor_matmul_i8(a, b, False))


def test_quantize(dev):
    a = np.array([0.25, 0.75, -0.25, 1000, -1000], np.float32)
    assert list(dev.tensor_quantize(a, 0.5)) == [0, 2, 0, 127, -127]
    rng = np.random.default_rng(3)
    x = awkward(rng, 200000, 60.0)
    x[:10] = [2.5, -2.5, 3.5, 126.5, 127.5, -127.5, np.inf, -np.inf, np.nan, -0.0]
    for k in (0.5, 0.37, 3.0, 1e-30):
        assert np.array_equal(dev.tensor_quantize(x, k), oracle.tensor_quantize(x, k)), k


def test_scale(dev):
    assert list(dev.tensor_scale(np.array([4, -6], np.int32), 0.5)) == [2.0, -3.0]
    rng = np.random.default_rng(4)
    i = rng.integers(-(1 << 31), 1 << 31, 100000, dtype=np.int64).astype(np.int32)
    assert np.array_equal(bits(dev.tensor_scale(i, 0.37)), bits(oracle.tensor_scale_i32(i, 0.37)))
    f = awkward(rng, 100000, 1e30)
    f[:3] = [np.inf, np.nan, -np.inf]
    want = (f * np.float32(0.0)).astype(np.float32)
    want[np.isnan(want)] = np.array([0x7FC00000], np.uint32).view(np.float32)[0]
    assert np.array_equal(bits(dev.tensor_scale(f, 0.0)), bits(want))


def test_argument_errors(dev):
    f = np.ones((2, 2), np.float32)
    with pytest.raises(rkhip.RKError) as e:
        dev.tensor_matmul(f, np.ones((3, 2), np.float32))
    assert e.value.code == -1
    L = rkhip.lib()
    c = np.empty(4, np.int32)
    i32 = np.ones(4, np.int32)
    # i32 inputs are rejected as by tenMatmul (tenErrArgs)
    assert L.rk_tensor_matmul(dev.h, rkhip.TENSOR_I32, 0, 2, 2, 2, rkhip._ptr(i32), rkhip._ptr(i32),
                              rkhip._ptr(c)) == -1
    with pytest.raises(rkhip.RKError):
        dev.tensor_quantize(f, 0.0)
    with pytest.raises(rkhip.RKError):
        dev.tensor_scale(np.ones(3, np.int8), 1.0)
