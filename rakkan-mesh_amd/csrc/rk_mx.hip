// rk_mx.hip — DeepSeek-V4.1 block-scaled ("microscaling") products on
// gfx950: the input quantized to E4M3 with a power-of-two scale per 32
// values (internal/num/mx.go:185-203 QuantizeActFP8), and products with
// E4M3 weights scaled per 32x32 block or packed E2M1 weights scaled per 32
// of a row (mx.go:282-334 MatVecFP8 / MatVecFP4, :371-388 combineBlocks).
//
// A block's 32 products sum exactly, so the block sum does not depend on
// its order:
//  * E4M3 x E4M3: each product has at most 8 significant bits and is a
//    multiple of 2^-18 below 2^18; the sum of 32 fits 41 bits, exact in
//    float64. The codes convert exactly in hardware (v_cvt_pk_f32_fp8, OCP
//    E4M3 on gfx950), then to float64, and the products go into float64
//    fused multiply-adds (full rate on CDNA4).
//  * E2M1 x E4M3: the reference's integer sum of twice the weight times
//    the input times 512 (an int32, wrapping). Here the weights convert to
//    float16 times 2^10 (v_cvt_scalef32_pk_f16_fp4) and the input to
//    float16, so each product is that integer, below 2^21.4; v_dot2_f32_f16
//    adds two of them, and a chain of two stays below 2^24, exact in
//    float32, before it is converted to an integer and added in int32.
//    An input block holding a NaN code (from an infinite or NaN input) adds,
//    as Go's int32(NaN) on x86-64 does, 0x80000000 for every odd twice-
//    weight at a NaN position.
// Then, as the CPU does it in float32: the block sum rounded to float32,
// times the input's scale, times the weight's, the blocks added in order,
// NaN canonical, rounded to bfloat16 (unless raw).
//
// Work layout: a workgroup takes RT rows; lane groups of LB lanes take one
// 32-weight block each (lane p of a group 32/LB consecutive weights), so a
// row's weights are read as one contiguous run by the workgroup, and each
// lane keeps its input slice in registers for all RT rows. The terms go to
// LDS, [row][block], and RT lanes of wave 0 add their rows' terms in block
// order (a sequential float32 chain, lds_chain_sum). Rows wider than the
// workgroup's blocks take several chunks, the chain carried across them.
#include <algorithm>
#include <mutex>

#include "rk_dev.h"
#include "rk_kernels.h"
#include "rk_mx.h"

namespace rk {

namespace {

typedef _Float16 rk_h2 __attribute__((ext_vector_type(2)));
typedef float rk_f2 __attribute__((ext_vector_type(2)));

constexpr float kInv448 = (float)(1.0 / 448);  // mx.go:40 inv448
constexpr float kActFloor = (float)1e-4;       // mx.go:42 actFloor
constexpr float kNaNf = __builtin_nanf("");

__device__ __forceinline__ float gomin(float x, float y) {
    if (x != x || y != y) return kNaNf;
    if (x < y) return x;
    if (y < x) return y;
    return u2f(f2u(x) | f2u(y));
}

// mx.go:147-156 pow2Ceil: the exponent field plus one if any mantissa bit
// is set (uint32 arithmetic, as the reference: a NaN gives 2^31, -0).
__device__ __forceinline__ float pow2ceil(float t) {
    const uint32_t b = f2u(t);
    const int32_t e = (int32_t)((b >> 23) & 0xff) - 127 + ((b & 0x7fffffu) ? 1 : 0);
    return u2f((uint32_t)(e + 127) << 23);
}

// mx.go:90-111 EncodeE4M3 of v within ±448, or NaN: below 2^-6 the
// multiples of 2^-9; else the exponent and the mantissa scaled to [8, 16),
// rounded to even (a carry to 16 moves to the next exponent).
__device__ __forceinline__ uint32_t encode_e4m3(float v) {
    if (v != v) return 0x7f;
    const uint32_t bits = f2u(v);
    const uint32_t sign = (bits >> 24) & 0x80;
    const uint32_t ab = bits & 0x7fffffffu;
    const float a = u2f(ab);
    if (a < 0.015625f) return sign | (uint32_t)rintf(a * 512.0f);
    int be = (int)(ab >> 23);                            // e + 127
    int n = (int)rintf(u2f((ab & 0x7fffffu) | (130u << 23)));  // [8, 16]
    if (n == 16) {
        be++;
        n = 8;
    }
    const int code = (be - 120) * 8 + (n - 8);  // (e+7)<<3 | (n-8)
    return sign | (uint32_t)min(code, 0x7e);
}

// mx.go:113-124 DecodeE8M0
__device__ __forceinline__ float e8m0(uint32_t c) {
    return c == 255 ? u2f(kCanonNaN) : c == 0 ? u2f(1u << 22) : u2f(c << 23);
}

// internal/num/matvec.go:22-29 ToBF16 then BF16 (RoundBF16)
__device__ __forceinline__ float round_bf16(float f) {
    const uint32_t b = f2u(f);
    if (f != f) return u2f(((b >> 16) | 0x40u) << 16);
    return u2f((b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u);
}

// mx.go:185-203: one lane per value, 32 lanes a block.
__global__ __launch_bounds__(256) void act_fp8_kernel(const float *x, int64_t n, uint8_t *codes, float *scales) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool in = i < n;  // n is a multiple of 32: whole blocks are in or out
    const float v = in ? x[i] : 0.0f;
    float m = fabsf(v);
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) m = gomax(m, __shfl_xor(m, o, 32));  // absMax (NaN if any)
    const float s = pow2ceil(gomax(m, kActFloor) * kInv448);
    const float q = __fdiv_rn(v, s);
    const uint32_t c = encode_e4m3(gomin(gomax(q, -448.0f), 448.0f));
    if (in) {
        codes[i] = (uint8_t)c;
        if ((threadIdx.x & 31) == 0) scales[i >> 5] = s;
    }
}

// E bytes a lane loads per row: 16, 8 or 4.
template <int E>
struct Chunk;
template <>
struct Chunk<16> {
    typedef uint4 T;
    static __device__ uint32_t word(const T &v, int k) { return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w; }
};
template <>
struct Chunk<8> {
    typedef uint2 T;
    static __device__ uint32_t word(const T &v, int k) { return k == 0 ? v.x : v.y; }
};
template <>
struct Chunk<4> {
    typedef uint32_t T;
    static __device__ uint32_t word(const T &v, int) { return v; }
};

// Terms per row in LDS: the workgroup's blocks, padded to keep rows 16-byte
// aligned and spread over the banks.
__device__ __host__ constexpr int term_stride(int cb) { return cb + 4; }

template <bool FP4, int LB, int RT>
__global__ __launch_bounds__(512) void mx_matvec_kernel(const uint8_t *__restrict__ w, const uint8_t *__restrict__ ws,
                                                        int64_t rows, int cols, const uint8_t *__restrict__ xc,
                                                        const float *__restrict__ xs, float *__restrict__ out,
                                                        int raw) {
    constexpr int NE = 32 / LB;               // weights (and inputs) per lane per row
    constexpr int WB = FP4 ? NE / 2 : NE;     // weight bytes per lane per row
    typedef Chunk<WB> WC;
    typedef typename WC::T WT;
    extern __shared__ __align__(16) float terms[];
    const int tid = threadIdx.x, p = tid % LB, bl = tid / LB;
    const int cb = blockDim.x / LB, ts = term_stride(cb);
    const int nb = cols >> 5;
    const int64_t row0 = (int64_t)blockIdx.x * RT;
    const int64_t rb = FP4 ? cols / 2 : cols;  // weight bytes per row
    float acc = 0.0f;                          // the chain of row row0 + tid (tid < RT)
    for (int c0 = 0; c0 < nb; c0 += cb) {       // uniform
        const int b = min(c0 + bl, nb - 1);     // past the last block: repeat it (its terms are not added)
        // the lane's input slice
        uint32_t xw[NE / 4];
#pragma unroll
        for (int k = 0; k < NE / 4; k++) xw[k] = *reinterpret_cast<const uint32_t *>(xc + b * 32 + p * NE + 4 * k);
        const float xsb = xs[b];
        // the rows' weights: all RT loads first, consumed in order
        WT wv[RT];
        uint32_t wsv[FP4 ? RT : 1];
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const int64_t rr = min(row0 + r, rows - 1);
            wv[r] = *reinterpret_cast<const WT *>(w + rr * rb + (int64_t)b * (FP4 ? 16 : 32) + p * WB);
            if constexpr (FP4) wsv[r] = ws[rr * nb + b];
        }
        float wsf = 0.0f;
        if constexpr (!FP4) wsf = e8m0(ws[(row0 >> 5) * nb + b]);  // RT divides 32: one scale row a tile
        if constexpr (!FP4) {
            double xv[NE];
#pragma unroll
            for (int k = 0; k < NE / 4; k++) {
                const rk_f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(xw[k], false);
                const rk_f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(xw[k], true);
                xv[4 * k] = lo.x, xv[4 * k + 1] = lo.y, xv[4 * k + 2] = hi.x, xv[4 * k + 3] = hi.y;
            }
#pragma unroll
            for (int r = 0; r < RT; r++) {
                double s0 = 0.0, s1 = 0.0;
#pragma unroll
                for (int k = 0; k < NE / 4; k++) {
                    const uint32_t u = WC::word(wv[r], k);
                    const rk_f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(u, false);
                    const rk_f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(u, true);
                    s0 = __builtin_fma((double)lo.x, xv[4 * k], s0);
                    s1 = __builtin_fma((double)lo.y, xv[4 * k + 1], s1);
                    s0 = __builtin_fma((double)hi.x, xv[4 * k + 2], s0);
                    s1 = __builtin_fma((double)hi.y, xv[4 * k + 3], s1);
                }
                double d = s0 + s1;  // exact: every partial sum is
#pragma unroll
                for (int o = 1; o < LB; o <<= 1) d += __shfl_xor(d, o);
                if (p == 0) {
                    float t = (float)d;
                    t = t * xsb;
                    t = t * wsf;
                    terms[r * ts + bl] = t;
                }
            }
        } else {
            // the input as float16 pairs; NaN codes as 0, their positions kept
            rk_h2 xh[NE / 2];
            uint32_t nanmask = 0;
#pragma unroll
            for (int k = 0; k < NE / 4; k++) {
                uint32_t u = xw[k];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (((u >> (8 * j)) & 0x7f) == 0x7f) {
                        nanmask |= 1u << (4 * k + j);
                        u &= ~(0xffu << (8 * j));
                    }
                xh[2 * k] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u, 1.0f, false);
                xh[2 * k + 1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u, 1.0f, true);
            }
#pragma unroll
            for (int r = 0; r < RT; r++) {
                uint32_t isum = 0;
#pragma unroll
                for (int k = 0; k < WB / 4; k++) {
                    const uint32_t u = WC::word(wv[r], k);  // 8 weights
                    const rk_h2 w0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1024.0f, 0);
                    const rk_h2 w1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1024.0f, 1);
                    const rk_h2 w2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1024.0f, 2);
                    const rk_h2 w3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1024.0f, 3);
                    const float f0 = __builtin_amdgcn_fdot2(w1, xh[4 * k + 1], __builtin_amdgcn_fdot2(w0, xh[4 * k], 0.0f, false), false);
                    const float f1 = __builtin_amdgcn_fdot2(w3, xh[4 * k + 3], __builtin_amdgcn_fdot2(w2, xh[4 * k + 2], 0.0f, false), false);
                    isum += (uint32_t)(int32_t)f0 + (uint32_t)(int32_t)f1;
                }
                if (nanmask) {  // rare: an infinite or NaN input in the block
                    uint32_t odd = 0;
#pragma unroll
                    for (int i = 0; i < NE; i++) {
                        const uint32_t nib = (WC::word(wv[r], i >> 3) >> (4 * (i & 7))) & 15u;
                        odd ^= ((nanmask >> i) & 1u) & (((nib & 5u) == 1u) ? 1u : 0u);
                    }
                    isum += odd << 31;
                }
#pragma unroll
                for (int o = 1; o < LB; o <<= 1) isum += (uint32_t)__shfl_xor((int)isum, o);
                if (p == 0) {
                    float t = (float)(int32_t)isum * 0.0009765625f;  // float32(sum / 1024): one rounding
                    t = t * xsb;
                    t = t * e8m0(wsv[r]);
                    terms[r * ts + bl] = t;
                }
            }
        }
        __syncthreads();
        if (tid < RT) acc = lds_chain_sum(terms + tid * ts, min(cb, nb - c0), acc);
        __syncthreads();  // the terms are read before the next chunk writes them
    }
    if (tid < RT && row0 + tid < rows) {
        const float v = canonical(acc);
        out[row0 + tid] = raw ? v : round_bf16(v);
    }
}

constexpr int kMxRows = 16;  // rows a workgroup (divides 32, the E4M3 scale rows)

template <bool FP4, int LB>
void launch_mx_t(const uint8_t *w, const uint8_t *ws, int64_t rows, int cols, const uint8_t *xc, const float *xs,
                 float *out, bool raw, int waves, hipStream_t s) {
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute((const void *)mx_matvec_kernel<FP4, LB, kMxRows>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    const int cb = 64 * waves / LB;
    const size_t lds = (size_t)kMxRows * term_stride(cb) * 4;
    const int64_t grid = (rows + kMxRows - 1) / kMxRows;
    RK_LAUNCH((mx_matvec_kernel<FP4, LB, kMxRows>), dim3((unsigned)grid), dim3((unsigned)(64 * waves)), lds, s, w, ws,
              rows, cols, xc, xs, out, raw ? 1 : 0);
}

// Lanes per block and waves per workgroup for nb blocks: the fewest idle
// lanes over the row's chunks, then the fewest chunks, then the widest
// loads.
void mx_shape(bool fp4, int nb, int *lb, int *waves) {
    const int cands8[3] = {2, 4, 8}, cands4[3] = {1, 2, 4};
    const int *c = fp4 ? cands4 : cands8;
    int64_t best = -1;
    for (int i = 0; i < 3; i++) {
        const int64_t lanes = (int64_t)nb * c[i];
        for (int W = 1; W <= 8; W++) {
            const int64_t per = 64 * W, chunks = (lanes + per - 1) / per;
            if (chunks * per - lanes >= per) continue;  // a whole idle wave
            const int64_t waste = chunks * per - lanes;
            const int64_t key = waste * 4096 + chunks * 16 + i;
            if (best < 0 || key < best) {
                best = key;
                *lb = c[i];
                *waves = W;
            }
        }
    }
}

}  // namespace

void launch_act_fp8(const float *x, int64_t n, uint8_t *codes, float *scales, hipStream_t s) {
    if (n <= 0) return;
    RK_LAUNCH(act_fp8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n, codes, scales);
}

void launch_mx_matvec(bool fp4, const uint8_t *w, const uint8_t *ws, int64_t rows, int64_t cols, const uint8_t *xc,
                      const float *xs, float *out, bool raw, hipStream_t s) {
    int lb = 2, waves = 1;
    mx_shape(fp4, (int)(cols / 32), &lb, &waves);
    if (fp4) {
        if (lb == 1) launch_mx_t<true, 1>(w, ws, rows, (int)cols, xc, xs, out, raw, waves, s);
        else if (lb == 2) launch_mx_t<true, 2>(w, ws, rows, (int)cols, xc, xs, out, raw, waves, s);
        else launch_mx_t<true, 4>(w, ws, rows, (int)cols, xc, xs, out, raw, waves, s);
    } else {
        if (lb == 2) launch_mx_t<false, 2>(w, ws, rows, (int)cols, xc, xs, out, raw, waves, s);
        else if (lb == 4) launch_mx_t<false, 4>(w, ws, rows, (int)cols, xc, xs, out, raw, waves, s);
        else launch_mx_t<false, 8>(w, ws, rows, (int)cols, xc, xs, out, raw, waves, s);
    }
}

}  // namespace rk
