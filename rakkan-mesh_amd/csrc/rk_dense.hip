// rk_dense.hip — float32 and bfloat16 matrix-vector products in the Dot32
// order (internal/num/matvec.go:32-67 Dot32 / DotBF16 / combine,
// :106-123 MatVec32 / MatVecBF16), for gfx950.
//
// Dot32 of a row: element i goes into running sum i mod 32, in order of i,
// each product rounded before it is added; then e_j = (s_j + s_j+8) +
// (s_j+16 + s_j+24) and ((e0+e1)+(e2+e3))+((e4+e5)+(e6+e7)). A bfloat16
// weight converts to float32 exactly, so DotBF16 is Dot32 of the converted
// row.
//
// Layout: rows padded with zeros to a multiple of 32 elements on upload
// (rk_matrix_upload). A padded element adds the product +0·+0 = +0 to its
// running sum, which leaves the sum unchanged: a sum starts at +0 and can
// never become -0 (x + y is -0 only when both are), so s + (+0) == s, NaN
// payloads included.
//
// Work layout: eight lanes per row; lane q of a row keeps the running sums
// 4q..4q+3 and at row step m (32 elements) reads elements 32m+4q..+3 (16
// bytes of float32 or 8 of bfloat16), so a row step is one 128- or 64-byte
// segment and a wave reads eight rows' segments per instruction. U steps
// of every row are in flight (a register ring): a wave keeps U·1 KiB
// (float32) in flight. The row's loads are buffer loads at a wave-uniform
// step offset; past the row's last step they repeat that step (cache hits)
// and those steps add +0, so every step issues the same loads and
// additions and the waits are fixed counts. The input is staged in LDS
// (zero-padded), in segments of kDenseMaxLdsElems for wider rows.
#include <algorithm>
#include <mutex>

#include "rk_dense.h"
#include "rk_dev.h"
#include "rk_kernels.h"

namespace rk {

namespace {

constexpr int kDenseU = 32;                 // row steps in flight per lane
constexpr int kDenseMaxLdsElems = 32768;    // input staged in LDS up to this width (128 KiB)
constexpr int64_t kDenseLaunchBytes = 1 << 30;  // a launch's matrix bytes (one buffer resource)

typedef int rk_v2i __attribute__((ext_vector_type(2)));

template <bool BF>
struct DenseStep {
    typedef rk_v4i type;
};
template <>
struct DenseStep<true> {
    typedef rk_v2i type;
};

template <bool BF>
__global__ __launch_bounds__(512) void dense_matvec_kernel(const void *w, int64_t rows, int row_elems,
                                                            const float *x, int cols, float *out) {
    typedef typename DenseStep<BF>::type V;
    extern __shared__ __align__(16) float sx[];
    constexpr int ES = BF ? 2 : 4;  // bytes per element
    constexpr int SB = 32 * ES;     // bytes per row step
    const int tid = threadIdx.x, lane = tid & 63, q = lane & 7;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (tid >> 6);
    const int64_t row = wave * 8 + (lane >> 3);
    // groups past the end repeat the last row (never stored) and take part
    // in the workgroup's barriers
    const int64_t r = row < rows ? row : rows - 1;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(w), 0, (int)(rows * row_elems * ES), kRsrcWord3);
    const int vo = (int)(r * row_elems * ES) + q * 4 * ES;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    // segments of the row whose input fits the LDS (one for widths up to
    // kDenseMaxLdsElems)
    for (int c0 = 0; c0 < row_elems; c0 += kDenseMaxLdsElems) {  // uniform
        const int ce = min(kDenseMaxLdsElems, row_elems - c0);
        const int nsteps = ce >> 5, mb = c0 >> 5;
        auto load = [&](int m) -> V {
            const int mm = mb + (m < nsteps ? m : nsteps - 1);
            if constexpr (BF)
                return __builtin_amdgcn_raw_buffer_load_b64(rs, vo, mm * SB, kAuxStream);
            else
                return __builtin_amdgcn_raw_buffer_load_b128(rs, vo, mm * SB, kAuxStream);
        };
        // the segment's first U steps, oldest first (the ring's waits count
        // on that order), then its input into LDS, zero past cols
        V wb[kDenseU];
#pragma unroll
        for (int u = 0; u < kDenseU; u++) {
            wb[u] = load(u);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c0 > 0) __syncthreads();  // every wave is done with the previous segment's input
        for (int i = tid; i < ce; i += blockDim.x) sx[i] = c0 + i < cols ? x[c0 + i] : 0.0f;
        __syncthreads();
        for (int m0 = 0; m0 < nsteps; m0 += kDenseU) {
#pragma unroll
            for (int u = 0; u < kDenseU; u++) {
                // every step adds (no branch, so no load is left in flight
                // under a register it is about to reload); a step past the
                // segment adds +0, which leaves the sum as it is
                const int m = m0 + u;
                const bool live = m < nsteps;  // uniform
                const float4 xv = reinterpret_cast<const float4 *>(sx)[(live ? m : nsteps - 1) * 8 + q];
                float4 wv;
                if constexpr (BF) {
                    const rk_v2i b = wb[u];
                    wv = make_float4(__int_as_float(b.x << 16), __int_as_float(b.x & (int)0xFFFF0000u),
                                     __int_as_float(b.y << 16), __int_as_float(b.y & (int)0xFFFF0000u));
                } else {
                    const rk_v4i b = wb[u];
                    wv = make_float4(__int_as_float(b.x), __int_as_float(b.y), __int_as_float(b.z),
                                     __int_as_float(b.w));
                }
                s0 += live ? wv.x * xv.x : 0.0f;
                s1 += live ? wv.y * xv.y : 0.0f;
                s2 += live ? wv.z * xv.z : 0.0f;
                s3 += live ? wv.w * xv.w : 0.0f;
                wb[u] = load(m + kDenseU);
            }
        }
    }
    // combine: lane q holds s_4q..s_4q+3; a = s_j + s_j+8 (lanes 0, 1) and
    // s_j+16 + s_j+24 (lanes 4, 5); e_j in lanes 0 (j < 4) and 1 (j >= 4)
    float a0 = s0 + __shfl_down(s0, 2, 8), a1 = s1 + __shfl_down(s1, 2, 8);
    float a2 = s2 + __shfl_down(s2, 2, 8), a3 = s3 + __shfl_down(s3, 2, 8);
    const float e0 = a0 + __shfl_down(a0, 4, 8), e1 = a1 + __shfl_down(a1, 4, 8);
    const float e2 = a2 + __shfl_down(a2, 4, 8), e3 = a3 + __shfl_down(a3, 4, 8);
    const float hsum = (e0 + e1) + (e2 + e3);
    const float res = hsum + __shfl_down(hsum, 1, 8);
    if (q == 0 && row < rows) out[row] = res;
}

template <bool BF>
void launch_dense_t(const void *w, int64_t rows, int row_elems, const float *x, int cols, float *out,
                    hipStream_t s) {
    const size_t lds = (size_t)std::min(row_elems, kDenseMaxLdsElems) * 4;
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute((const void *)dense_matvec_kernel<BF>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  kDenseMaxLdsElems * 4);
    });
    const int64_t waves = (rows + 7) / 8;
    // up to 8 waves (two a SIMD: the ring's registers allow no more)
    const int64_t W = std::min<int64_t>(8, std::max<int64_t>(1, (waves + 255) / 256));
    const int64_t grid = (waves + W - 1) / W;
    RK_LAUNCH((dense_matvec_kernel<BF>), dim3((unsigned)grid), dim3((unsigned)(64 * W)), lds, s, w, rows, row_elems,
              x, cols, out);
}

}  // namespace

int64_t dense_row_elems(int64_t cols) { return (cols + 31) & ~(int64_t)31; }

void launch_dense_matvec(bool bf16, const void *w, int64_t rows, int64_t cols, const float *x, float *out,
                         hipStream_t s) {
    const int row_elems = (int)dense_row_elems(cols);
    const int64_t rb = (int64_t)row_elems * (bf16 ? 2 : 4);
    const int64_t per = std::max<int64_t>(1, kDenseLaunchBytes / rb);  // rows of one launch
    for (int64_t r0 = 0; r0 < rows; r0 += per) {
        const int64_t n = std::min(per, rows - r0);
        const void *wr = static_cast<const uint8_t *>(w) + r0 * rb;
        if (bf16)
            launch_dense_t<true>(wr, n, row_elems, x, (int)cols, out + r0, s);
        else
            launch_dense_t<false>(wr, n, row_elems, x, (int)cols, out + r0, s);
    }
}

}  // namespace rk
