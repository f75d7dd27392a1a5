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
// Work layout: 32/SL lanes per row; lane l of a row keeps the running sums
// SL·l .. SL·l+SL-1 and at row step m (32 elements) reads elements
// 32m+SL·l .. +SL-1, so a row step is one contiguous 128-byte (float32) or
// 64-byte (bfloat16) segment. U steps of every row are in flight (a
// register ring). The row's loads are buffer loads at a wave-uniform step
// offset; past the row's last step they repeat that step (cache hits) and
// those steps add +0, so every step issues the same loads and additions and
// the waits are fixed counts. The input is staged in LDS (zero-padded), in
// segments of kDenseMaxLdsElems for wider rows, and read a block of U steps
// at a time.
#include <algorithm>
#include <mutex>

#include "rk_dense.h"
#include "rk_dev.h"
#include "rk_kernels.h"

namespace rk {

namespace {

// Running sums per lane (32/SL lanes a row) and row steps in flight, the
// fastest measured on MI355X: float32 one sum a lane (4-byte loads, two
// rows a wave), bfloat16 two (one 4-byte word, four rows a wave).
constexpr int kDenseSlF32 = 1;
constexpr int kDenseSlBf16 = 2;
constexpr int kDenseU = 16;
constexpr int kDenseMaxLdsElems = 32768;    // input staged in LDS up to this width (128 KiB)
constexpr int64_t kDenseLaunchBytes = 1 << 30;  // a launch's matrix bytes (one buffer resource)

typedef int rk_v2i __attribute__((ext_vector_type(2)));

// Lanes per row 32/SL: lane l of a row keeps running sums SL·l .. SL·l+SL-1
// and reads SL elements per row step. U row steps in flight (U <= 63, the
// vector memory counter's range).
template <bool BF, int SL>
struct DenseLoad;
template <>
struct DenseLoad<false, 1> {
    typedef int type;
    static __device__ type load(__amdgpu_buffer_rsrc_t r, int v, int s) {
        return __builtin_amdgcn_raw_buffer_load_b32(r, v, s, kAuxStream);
    }
};
template <>
struct DenseLoad<false, 2> {
    typedef rk_v2i type;
    static __device__ type load(__amdgpu_buffer_rsrc_t r, int v, int s) {
        return __builtin_amdgcn_raw_buffer_load_b64(r, v, s, kAuxStream);
    }
};
template <>
struct DenseLoad<false, 4> {
    typedef rk_v4i type;
    static __device__ type load(__amdgpu_buffer_rsrc_t r, int v, int s) {
        return __builtin_amdgcn_raw_buffer_load_b128(r, v, s, kAuxStream);
    }
};
template <>
struct DenseLoad<true, 2> {
    typedef int type;
    static __device__ type load(__amdgpu_buffer_rsrc_t r, int v, int s) {
        return __builtin_amdgcn_raw_buffer_load_b32(r, v, s, kAuxStream);
    }
};
template <>
struct DenseLoad<true, 4> {
    typedef rk_v2i type;
    static __device__ type load(__amdgpu_buffer_rsrc_t r, int v, int s) {
        return __builtin_amdgcn_raw_buffer_load_b64(r, v, s, kAuxStream);
    }
};

// Element k (< SL) of a loaded step as float32.
template <bool BF, int SL, typename V>
__device__ __forceinline__ float dense_elem(const V &v, int k) {
    if constexpr (!BF) {
        if constexpr (SL == 1)
            return __int_as_float(v);
        else
            return __int_as_float(v[k]);
    } else {
        int word;
        if constexpr (SL == 2)
            word = v;
        else
            word = v[k >> 1];
        return __int_as_float((k & 1) ? (word & (int)0xFFFF0000u) : (word << 16));
    }
}

template <bool BF, int SL, int U>
__global__ __launch_bounds__(512) void dense_matvec_kernel(const void *w, int64_t rows, int row_elems,
                                                            const float *x, int cols, float *out) {
    typedef DenseLoad<BF, SL> LD;
    typedef typename LD::type V;
    constexpr int LPR = 32 / SL;    // lanes per row
    constexpr int RPW = 64 / LPR;   // rows per wave
    constexpr int ES = BF ? 2 : 4;  // bytes per element
    constexpr int SB = 32 * ES;     // bytes per row step
    extern __shared__ __align__(16) float sx[];
    const int tid = threadIdx.x, lane = tid & 63, l = lane % LPR;
    const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (tid >> 6);
    const int64_t row = wave * RPW + lane / LPR;
    // groups past the end repeat the last row (never stored) and take part
    // in the workgroup's barriers
    const int64_t r = row < rows ? row : rows - 1;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(w), 0, (int)(rows * row_elems * ES), kRsrcWord3);
    const int vo = (int)(r * row_elems * ES) + l * SL * ES;
    float acc[SL];
#pragma unroll
    for (int k = 0; k < SL; k++) acc[k] = 0.0f;
    // segments of the row whose input fits the LDS (one for widths up to
    // kDenseMaxLdsElems)
    for (int c0 = 0; c0 < row_elems; c0 += kDenseMaxLdsElems) {  // uniform
        const int ce = min(kDenseMaxLdsElems, row_elems - c0);
        const int nsteps = ce >> 5, mb = c0 >> 5;
        auto load = [&](int m) -> V { return LD::load(rs, vo, (mb + (m < nsteps ? m : nsteps - 1)) * SB); };
        // the segment's first U steps, oldest first (the ring's waits count
        // on that order), then its input into LDS, zero past cols
        V wb[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            wb[u] = load(u);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c0 > 0) __syncthreads();  // every wave is done with the previous segment's input
        for (int i = tid; i < ce; i += blockDim.x) sx[i] = c0 + i < cols ? x[c0 + i] : 0.0f;
        __syncthreads();
        for (int m0 = 0; m0 < nsteps; m0 += U) {
            // the block's U input steps from LDS first (one LDS latency a
            // block, not a step)
            float xv[U][SL];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int m = m0 + u;
                const float *xp = sx + (m < nsteps ? m : nsteps - 1) * 32 + l * SL;
                if constexpr (SL == 4) {
                    const float4 t = *reinterpret_cast<const float4 *>(xp);
                    xv[u][0] = t.x, xv[u][1] = t.y, xv[u][2] = t.z, xv[u][3] = t.w;
                } else if constexpr (SL == 2) {
                    const float2 t = *reinterpret_cast<const float2 *>(xp);
                    xv[u][0] = t.x, xv[u][1] = t.y;
                } else {
                    xv[u][0] = xp[0];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < U; u++) {
                // every step adds (no branch, so no load is left in flight
                // under a register it is about to reload); a step past the
                // segment adds +0, which leaves the sum as it is
                const int m = m0 + u;
                const bool live = m < nsteps;  // uniform
#pragma unroll
                for (int k = 0; k < SL; k++)
                    acc[k] += live ? dense_elem<BF, SL>(wb[u], k) * xv[u][k] : 0.0f;
                wb[u] = load(m + U);
            }
        }
    }
    // Dot32's combine: s_j sits in lane j/SL of the row, element j mod SL.
    // a = s_j + s_j+8 (lanes of j < 8), then + (s_j+16 + s_j+24) gives e_j;
    // then ((e0+e1)+(e2+e3))+((e4+e5)+(e6+e7)).
    float e[SL];
#pragma unroll
    for (int k = 0; k < SL; k++) {
        const float a = acc[k] + __shfl_down(acc[k], 8 / SL, LPR);
        e[k] = a + __shfl_down(a, 16 / SL, LPR);
    }
    // lanes 0 .. 8/SL-1 hold e_j (j = SL·l + k)
    float res;
    if constexpr (SL == 4) {
        const float h = (e[0] + e[1]) + (e[2] + e[3]);  // lane 0: e0..e3; lane 1: e4..e7
        res = h + __shfl_down(h, 1, LPR);
    } else if constexpr (SL == 2) {
        const float p = e[0] + e[1];                    // lane l: e_2l + e_2l+1
        const float t = p + __shfl_down(p, 1, LPR);     // lanes 0, 2
        res = t + __shfl_down(t, 2, LPR);
    } else {
        const float p = e[0] + __shfl_down(e[0], 1, LPR);  // lanes 0, 2, 4, 6
        const float t = p + __shfl_down(p, 2, LPR);        // lanes 0, 4
        res = t + __shfl_down(t, 4, LPR);
    }
    if (l == 0 && row < rows) out[row] = res;
}

template <bool BF, int SL, int U>
void launch_dense_t(const void *w, int64_t rows, int row_elems, const float *x, int cols, float *out,
                    hipStream_t s, int waves_per_wg = 0) {
    constexpr int RPW = 2 * SL;
    const size_t lds = (size_t)std::min(row_elems, kDenseMaxLdsElems) * 4;
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute((const void *)dense_matvec_kernel<BF, SL, U>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kDenseMaxLdsElems * 4);
    });
    const int64_t waves = (rows + RPW - 1) / RPW;
    // four waves a workgroup once there are enough (measured best on
    // MI355X for 4096- and 14336-row products)
    const int64_t W = waves_per_wg > 0 ? waves_per_wg : std::min<int64_t>(4, std::max<int64_t>(1, waves / 256));
    const int64_t grid = (waves + W - 1) / W;
    RK_LAUNCH((dense_matvec_kernel<BF, SL, U>), dim3((unsigned)grid), dim3((unsigned)(64 * W)), lds, s, w, rows,
              row_elems, x, cols, out);
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
            launch_dense_t<true, kDenseSlBf16, kDenseU>(wr, n, row_elems, x, (int)cols, out + r0, s);
        else
            launch_dense_t<false, kDenseSlF32, kDenseU>(wr, n, row_elems, x, (int)cols, out + r0, s);
    }
}

}  // namespace rk
