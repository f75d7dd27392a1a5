// rk_tensor.hip — the rakkan_tensor_v1 operators on this path
// (internal/sandbox/tensor.go): matmul / matmul_t in f32 and i8, and the
// quantize / scale that produce and consume the i8 form.
//
// f32 (tensor.go:318-327): c_ij = Canonical(acc), acc += float32(a_ip·b_pj)
// for p = 0..k-1 from +0 — a sequential sum per output, so each output is
// one lane's chain of multiplies and adds on the vector ALUs (a matrix
// core's reduction tree would round differently). A workgroup stages
// 64-position slices of its 32 rows of a and 32 columns of b in LDS (b as
// columns, so both read four positions per 16-byte load) and each thread
// runs four chains (2 rows x 2 columns).
//
// i8 (tensor.go:328-335): c_ij = Σ int32(a_ip)·int32(b_pj) with Go's int32
// wraparound. Integer sums are exact in any order, so the block sums run on
// int8 MFMA (v_mfma_i32_16x16x32_i8, accumulator chained); the accumulator
// restarts every 65536 positions (|partial| <= 2^30, no overflow inside the
// matrix core) and the partials are added with wrapping integer adds.
#include <algorithm>
#include <mutex>

#include "rk_dev.h"
#include "rk_kernels.h"
#include "rk_runtime.h"

namespace rk {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---- f32 ----
constexpr int kTfTile = 32;    // outputs per side of a workgroup
constexpr int kTfChunk = 64;   // positions per staged slice
constexpr int kTfPitch = kTfChunk + 4;

__global__ __launch_bounds__(256) void tensor_mm_f32_kernel(const float *a, const float *b, float *c, int64_t m,
                                                            int64_t k, int64_t n, int transposed) {
    __shared__ __align__(16) float sa[kTfTile][kTfPitch];  // rows of a
    __shared__ __align__(16) float sb[kTfTile][kTfPitch];  // columns of b
    const int tid = threadIdx.x;
    const int64_t i0 = (int64_t)blockIdx.y * kTfTile, j0 = (int64_t)blockIdx.x * kTfTile;
    // thread -> rows i0 + ti, i0 + ti + 16 and columns j0 + tj, j0 + tj + 16
    const int ti = tid >> 4, tj = tid & 15;
    float acc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
    for (int64_t p0 = 0; p0 < k; p0 += kTfChunk) {
        const int np = (int)min((int64_t)kTfChunk, k - p0);
        // stage: 32 x 64 of each (zeros past k are never summed)
        for (int e = tid; e < kTfTile * kTfChunk; e += 256) {
            const int r = e / kTfChunk, p = e % kTfChunk;
            const int64_t gi = min(i0 + r, m - 1), gp = min(p0 + p, k - 1);
            sa[r][p] = a[gi * k + gp];
        }
        if (transposed) {  // b[n][k]: column j of the product is row j
            for (int e = tid; e < kTfTile * kTfChunk; e += 256) {
                const int r = e / kTfChunk, p = e % kTfChunk;
                const int64_t gj = min(j0 + r, n - 1), gp = min(p0 + p, k - 1);
                sb[r][p] = b[gj * k + gp];
            }
        } else {  // b[k][n]: read along n, store as columns
            for (int e = tid; e < kTfTile * kTfChunk; e += 256) {
                const int p = e / kTfTile, r = e % kTfTile;
                const int64_t gj = min(j0 + r, n - 1), gp = min(p0 + p, k - 1);
                sb[r][p] = b[gp * n + gj];
            }
        }
        __syncthreads();
        const float *ra0 = sa[ti], *ra1 = sa[ti + 16], *rb0 = sb[tj], *rb1 = sb[tj + 16];
        int p = 0;
        for (; p + 4 <= np; p += 4) {
            const float4 x0 = *reinterpret_cast<const float4 *>(ra0 + p);
            const float4 x1 = *reinterpret_cast<const float4 *>(ra1 + p);
            const float4 y0 = *reinterpret_cast<const float4 *>(rb0 + p);
            const float4 y1 = *reinterpret_cast<const float4 *>(rb1 + p);
            const float xa[2][4] = {{x0.x, x0.y, x0.z, x0.w}, {x1.x, x1.y, x1.z, x1.w}};
            const float yb[2][4] = {{y0.x, y0.y, y0.z, y0.w}, {y1.x, y1.y, y1.z, y1.w}};
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int r = 0; r < 2; r++)
#pragma unroll
                    for (int s = 0; s < 2; s++) acc[r][s] += xa[r][q] * yb[s][q];
        }
        for (; p < np; p++)
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int s = 0; s < 2; s++) acc[r][s] += sa[ti + 16 * r][p] * sb[tj + 16 * s][p];
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int64_t i = i0 + ti + 16 * r, j = j0 + tj + 16 * s;
            if (i < m && j < n) c[i * n + j] = canonical(acc[r][s]);
        }
}

// ---- i8 ----
constexpr int kTiTile = 64;    // outputs per side of a workgroup
constexpr int kTiChunk = 256;  // positions per staged slice
constexpr int kTiPitch = kTiChunk + 8;  // bytes: 16 rows at one offset in distinct banks
constexpr int64_t kTiRestart = 65536;   // positions per matrix-core accumulation

__global__ __launch_bounds__(256) void tensor_mm_i8_kernel(const int8_t *a, const int8_t *b, int32_t *c, int64_t m,
                                                           int64_t k, int64_t n, int transposed) {
    __shared__ __align__(16) int8_t sa[kTiTile][kTiPitch];  // rows of a
    __shared__ __align__(16) int8_t sb[kTiTile][kTiPitch];  // columns of b
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lq = lane >> 4, ln = lane & 15;
    const int wr = wave & 1, wc = wave >> 1;  // the wave's 32 x 32 quarter
    const int64_t i0 = (int64_t)blockIdx.y * kTiTile, j0 = (int64_t)blockIdx.x * kTiTile;
    v4i d[2][2];
    int32_t tot[2][2][4];
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int s = 0; s < 2; s++) {
            d[r][s] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 4; e++) tot[r][s][e] = 0;
        }
    for (int64_t p0 = 0; p0 < k; p0 += kTiChunk) {
        // stage 64 x 256 of each; positions past k are zeros (they add 0)
        for (int e = tid; e < kTiTile * (kTiChunk / 4); e += 256) {
            const int r = e / (kTiChunk / 4), p = 4 * (e % (kTiChunk / 4));
            const int64_t gi = min(i0 + r, m - 1);
            uint32_t w = 0;
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (p0 + p + q < k) w |= (uint32_t)(uint8_t)a[gi * k + p0 + p + q] << (8 * q);
            *reinterpret_cast<uint32_t *>(&sa[r][p]) = w;
        }
        if (transposed) {
            for (int e = tid; e < kTiTile * (kTiChunk / 4); e += 256) {
                const int r = e / (kTiChunk / 4), p = 4 * (e % (kTiChunk / 4));
                const int64_t gj = min(j0 + r, n - 1);
                uint32_t w = 0;
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (p0 + p + q < k) w |= (uint32_t)(uint8_t)b[gj * k + p0 + p + q] << (8 * q);
                *reinterpret_cast<uint32_t *>(&sb[r][p]) = w;
            }
        } else {
            for (int e = tid; e < kTiTile * (kTiChunk / 4); e += 256) {
                const int r = e % kTiTile, p = 4 * (e / kTiTile);
                const int64_t gj = min(j0 + r, n - 1);
                uint32_t w = 0;
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (p0 + p + q < k) w |= (uint32_t)(uint8_t)b[(p0 + p + q) * n + gj] << (8 * q);
                *reinterpret_cast<uint32_t *>(&sb[r][p]) = w;
            }
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < kTiChunk / 32; ks++) {
            long fa[2], fb[2];
#pragma unroll
            for (int r = 0; r < 2; r++)
                fa[r] = *reinterpret_cast<const long *>(&sa[32 * wr + 16 * r + ln][32 * ks + 8 * lq]);
#pragma unroll
            for (int s = 0; s < 2; s++)
                fb[s] = *reinterpret_cast<const long *>(&sb[32 * wc + 16 * s + ln][32 * ks + 8 * lq]);
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int s = 0; s < 2; s++) d[r][s] = __builtin_amdgcn_mfma_i32_16x16x32_i8(fa[r], fb[s], d[r][s], 0, 0, 0);
        }
        __syncthreads();
        if ((p0 + kTiChunk) % kTiRestart == 0 || p0 + kTiChunk >= k) {
            // fold the matrix core's partial into the wrapping total
#pragma unroll
            for (int r = 0; r < 2; r++)
#pragma unroll
                for (int s = 0; s < 2; s++) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        tot[r][s][e] = (int32_t)((uint32_t)tot[r][s][e] + (uint32_t)d[r][s][e]);
                    d[r][s] = v4i{0, 0, 0, 0};
                }
        }
    }
    // the 16x16 result layout: lane holds column ln, rows 4·lq + e
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int64_t j = j0 + 32 * wc + 16 * s + ln;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int64_t i = i0 + 32 * wr + 16 * r + 4 * lq + e;
                if (i < m && j < n) c[i * n + j] = tot[r][s][e];
            }
        }
}

// ---- elementwise ----
// tensor.go:445-461: q = int8(max(-127, min(127, float32(RoundToEven(v/k)))))
// with v/k the correctly rounded f32 quotient; NaN quotients give 0 (Go's
// conversion of NaN on amd64 takes the low byte of 0x80000000).
__global__ void tensor_quantize_kernel(const float *a, int8_t *q, int64_t n, float k) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float r = __builtin_rintf(a[i] / k);
        q[i] = (int8_t)(r != r ? 0 : (r > 127.0f ? 127 : (r < -127.0f ? -127 : (int)r)));
    }
}

// tensor.go:366-387: out = Canonical(float32(v)·k), v f32 or i32.
__global__ void tensor_scale_kernel(const void *a, int i32, float *out, int64_t n, float k) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float v = i32 ? (float)static_cast<const int32_t *>(a)[i] : static_cast<const float *>(a)[i];
        out[i] = canonical(v * k);
    }
}

}  // namespace

int enqueue_tensor_matmul(rk_device *d, int32_t dtype, int32_t transposed, int64_t m, int64_t k, int64_t n,
                          const void *a, const void *b, void *c, hipStream_t s) {
    if (dtype == RK_TENSOR_F32) {
        const dim3 grid((unsigned)((n + kTfTile - 1) / kTfTile), (unsigned)((m + kTfTile - 1) / kTfTile));
        ProfScope p(d, s, "tensor_matmul_f32");
        RK_LAUNCH(tensor_mm_f32_kernel, grid, dim3(256), 0, s, static_cast<const float *>(a),
                  static_cast<const float *>(b), static_cast<float *>(c), m, k, n, transposed ? 1 : 0);
    } else {
        const dim3 grid((unsigned)((n + kTiTile - 1) / kTiTile), (unsigned)((m + kTiTile - 1) / kTiTile));
        ProfScope p(d, s, "tensor_matmul_i8");
        RK_LAUNCH(tensor_mm_i8_kernel, grid, dim3(256), 0, s, static_cast<const int8_t *>(a),
                  static_cast<const int8_t *>(b), static_cast<int32_t *>(c), m, k, n, transposed ? 1 : 0);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(d, e, "tensor matmul launch");
    return RK_OK;
}

static unsigned elem_grid(int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 65536); }

int enqueue_tensor_quantize(rk_device *d, const float *a, int8_t *q, int64_t n, float k, hipStream_t s) {
    ProfScope p(d, s, "tensor_quantize");
    RK_LAUNCH(tensor_quantize_kernel, dim3(elem_grid(n)), dim3(256), 0, s, a, q, n, k);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? RK_OK : hip_fail(d, e, "tensor quantize launch");
}

int enqueue_tensor_scale(rk_device *d, int32_t dtype, const void *a, float *out, int64_t n, float k, hipStream_t s) {
    ProfScope p(d, s, "tensor_scale");
    RK_LAUNCH(tensor_scale_kernel, dim3(elem_grid(n)), dim3(256), 0, s, a, dtype == RK_TENSOR_I32 ? 1 : 0, out, n, k);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? RK_OK : hip_fail(d, e, "tensor scale launch");
}

}  // namespace rk

using namespace rk;

namespace {

// Shape and type checks of tenMatmul (tensor.go:287-300): the same dtype on
// both sides, not i32; dimensions within the tensor table's 2^24 limit
// (tensor.go:60).
int check_tensor_matmul(rk_device *d, int32_t dtype, int64_t m, int64_t k, int64_t n) {
    if (!d) return RK_ERR_ARGS;
    if (dtype != RK_TENSOR_F32 && dtype != RK_TENSOR_I8)
        return fail(d, RK_ERR_ARGS, "rk_tensor_matmul: dtype %d (f32 or i8 only)", dtype);
    const int64_t lim = (int64_t)1 << 24;
    if (m <= 0 || k <= 0 || n <= 0 || m > lim || k > lim || n > lim)
        return fail(d, RK_ERR_ARGS, "rk_tensor_matmul: shape %lldx%lld by %lld", (long long)m, (long long)k,
                    (long long)n);
    return RK_OK;
}

size_t dsize(int32_t dtype) { return dtype == RK_TENSOR_I8 ? 1 : 4; }

}  // namespace

extern "C" {

int rk_tensor_matmul(rk_device *d, int32_t dtype, int32_t transposed, int64_t m, int64_t k, int64_t n, const void *a,
                     const void *b, void *c) {
    int rc = check_tensor_matmul(d, dtype, m, k, n);
    if (rc) return rc;
    if (!a || !b || !c) return fail(d, RK_ERR_ARGS, "rk_tensor_matmul: null buffer");
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    if (d->capturing) return fail(d, RK_ERR_ARGS, "rk_tensor_matmul waits for its result: it cannot be recorded");
    const size_t ab = (size_t)(m * k) * dsize(dtype), bb = (size_t)(k * n) * dsize(dtype), cb = (size_t)(m * n) * 4;
    void *da = nullptr, *db = nullptr, *dc = nullptr;
    if ((rc = dev_alloc(d, &da, ab, "tensor a")) || (rc = dev_alloc(d, &db, bb, "tensor b")) ||
        (rc = dev_alloc(d, &dc, cb, "tensor c"))) {
        (void)hipFree(da);
        (void)hipFree(db);
        return rc;
    }
    hipStream_t s = d->stream;
    hipError_t e = hipMemcpyAsync(da, a, ab, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(db, b, bb, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) rc = enqueue_tensor_matmul(d, dtype, transposed, m, k, n, da, db, dc, s);
    if (e == hipSuccess && !rc) e = hipMemcpyAsync(c, dc, cb, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && !rc) e = hipStreamSynchronize(s);
    (void)hipFree(da);
    (void)hipFree(db);
    (void)hipFree(dc);
    if (rc) return rc;
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return hip_fail(d, e, "rk_tensor_matmul");
    }
    return RK_OK;
}

int rk_tensor_matmul_device(rk_device *d, int32_t dtype, int32_t transposed, int64_t m, int64_t k, int64_t n,
                            const void *d_a, const void *d_b, void *d_c, void *stream) {
    int rc = check_tensor_matmul(d, dtype, m, k, n);
    if (rc) return rc;
    if (!d_a || !d_b || !d_c) return fail(d, RK_ERR_ARGS, "rk_tensor_matmul_device: null buffer");
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    hipStream_t s = stream ? (hipStream_t)stream : d->stream;
    if (d->capturing && s != d->stream)
        return fail(d, RK_ERR_ARGS, "while recording a graph, work goes on the device's stream");
    return enqueue_tensor_matmul(d, dtype, transposed, m, k, n, d_a, d_b, d_c, s);
}

int rk_tensor_quantize(rk_device *d, const float *a, int8_t *q, int64_t n, float k) {
    if (!d) return RK_ERR_ARGS;
    if (!(k > 0.0f) || n < 0 || (n > 0 && (!a || !q))) return fail(d, RK_ERR_ARGS, "rk_tensor_quantize: bad arguments");
    if (n == 0) return RK_OK;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    if (d->capturing) return fail(d, RK_ERR_ARGS, "rk_tensor_quantize waits for its result: it cannot be recorded");
    float *da = nullptr;
    int8_t *dq = nullptr;
    int rc;
    if ((rc = dev_alloc(d, (void **)&da, (size_t)n * 4, "tensor")) || (rc = dev_alloc(d, (void **)&dq, (size_t)n, "tensor"))) {
        (void)hipFree(da);
        return rc;
    }
    hipStream_t s = d->stream;
    hipError_t e = hipMemcpyAsync(da, a, (size_t)n * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) rc = enqueue_tensor_quantize(d, da, dq, n, k, s);
    if (e == hipSuccess && !rc) e = hipMemcpyAsync(q, dq, (size_t)n, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && !rc) e = hipStreamSynchronize(s);
    (void)hipFree(da);
    (void)hipFree(dq);
    if (rc) return rc;
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return hip_fail(d, e, "rk_tensor_quantize");
    }
    return RK_OK;
}

int rk_tensor_scale(rk_device *d, int32_t dtype, const void *a, float *out, int64_t n, float k) {
    if (!d) return RK_ERR_ARGS;
    if ((dtype != RK_TENSOR_F32 && dtype != RK_TENSOR_I32) || n < 0 || (n > 0 && (!a || !out)))
        return fail(d, RK_ERR_ARGS, "rk_tensor_scale: bad arguments (f32 or i32 input)");
    if (n == 0) return RK_OK;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    if (d->capturing) return fail(d, RK_ERR_ARGS, "rk_tensor_scale waits for its result: it cannot be recorded");
    void *da = nullptr;
    float *dout = nullptr;
    int rc;
    if ((rc = dev_alloc(d, &da, (size_t)n * 4, "tensor")) || (rc = dev_alloc(d, (void **)&dout, (size_t)n * 4, "tensor"))) {
        (void)hipFree(da);
        return rc;
    }
    hipStream_t s = d->stream;
    hipError_t e = hipMemcpyAsync(da, a, (size_t)n * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) rc = enqueue_tensor_scale(d, dtype, da, dout, n, k, s);
    if (e == hipSuccess && !rc) e = hipMemcpyAsync(out, dout, (size_t)n * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && !rc) e = hipStreamSynchronize(s);
    (void)hipFree(da);
    (void)hipFree(dout);
    if (rc) return rc;
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return hip_fail(d, e, "rk_tensor_scale");
    }
    return RK_OK;
}

}  // extern "C"
