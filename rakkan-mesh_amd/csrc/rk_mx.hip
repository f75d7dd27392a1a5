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
// Work layout: lane groups of LB lanes take one 32-weight block each (lane
// p of a group 32/LB consecutive weights: 16-byte loads), so a row's
// weights are read as one contiguous run, and each lane keeps its input
// slice in registers for all the workgroup's rows. A workgroup takes RT = 8
// row steps; narrow rows go G side by side (G runs of 8 consecutive rows,
// a step reading one row of each run), all RT loads issued before the first
// is used. The terms go to LDS, [row][block], and one lane per row adds
// them in block order (a sequential float32 chain, lds_chain_sum). Rows
// wider than the workgroup's lanes take several chunks, the chain carried
// across them. With a slot table the grid's second dimension runs selected
// experts (ExpertMatVecs). Also here: the in-place E4M3 / E2M1 quantizers
// of the DeepSeek batch (ActQuantInPlace, FP4QuantInPlace).
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
    // v / s: v times 1/s where s is a normal power of two (one rounding
    // either way); a division for the scales of blocks with infinities or
    // NaNs (+inf, -0)
    const uint32_t e = f2u(s) >> 23;  // 256 for -0
    float q;
    if (e >= 1 && e <= 253)
        q = v * u2f((254u - e) << 23);
    else
        q = __fdiv_rn(v, s);
    const uint32_t c = encode_e4m3(gomin(gomax(q, -448.0f), 448.0f));
    if (in) {
        codes[i] = (uint8_t)c;
        if ((threadIdx.x & 31) == 0) scales[i >> 5] = s;
    }
}

// internal/gpu/mx.go:146-172 actFP8Kernel's arena form of the codes: each
// code's value, unscaled, as a float32 word (exact: E4M3 values are
// float32 values).
__global__ __launch_bounds__(256) void e4m3_values_kernel(const uint8_t *codes, int64_t n, float *out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = __builtin_amdgcn_cvt_pk_f32_fp8((uint32_t)codes[i], false)[0];
}

// mx.go:205-214 ActQuantInPlace: each value its E4M3 rounding (as
// act_fp8_kernel) times the block scale, rounded to bfloat16.
__global__ __launch_bounds__(256) void act_quant_inplace_kernel(float *x, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool in = i < n;
    const float v = in ? x[i] : 0.0f;
    float m = fabsf(v);
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) m = gomax(m, __shfl_xor(m, o, 32));
    const float s = pow2ceil(gomax(m, kActFloor) * kInv448);
    const uint32_t c = encode_e4m3(gomin(gomax(__fdiv_rn(v, s), -448.0f), 448.0f));
    const float q = __builtin_amdgcn_cvt_pk_f32_fp8(c, false)[0];  // the code's value, exact
    if (in) x[i] = round_bf16(q * s);
}

// mx.go:128-145 EncodeE2M1: the nearest of 0, .5, 1, 1.5, 2, 3, 4, 6, ties
// to the even code; the sign kept (NaN: code 0 and its sign).
__device__ __forceinline__ uint32_t encode_e2m1(float v) {
    const float a = fabsf(v);
    const float mid[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
    uint32_t code = 0;
#pragma unroll
    for (int k = 0; k < 7; k++)
        if (a > mid[k] || (a == mid[k] && ((k + 1) & 1) == 0)) code = (uint32_t)(k + 1);
    return code | ((f2u(v) >> 31) << 3);
}

// mx.go:234-280 QuantizeFP4 then DequantFP4 (FP4QuantInPlace): blocks of 16
// with an E4M3 scale of amax/6 (E4M3 = true), or of 32 with the power of
// two pow2Ceil(amax/6) stored as its exponent byte; each value becomes its
// E2M1 code's value times the stored scale, rounded to bfloat16.
template <bool E4M3>
__global__ __launch_bounds__(256) void fp4_quant_inplace_kernel(float *x, int64_t n) {
    constexpr int BS = E4M3 ? 16 : 32;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool in = i < n;
    const float v = in ? x[i] : 0.0f;
    float m = fabsf(v);
#pragma unroll
    for (int o = 1; o < BS; o <<= 1) m = gomax(m, __shfl_xor(m, o, BS));
    float s, stored;
    if constexpr (E4M3) {
        m = gomax(m, 0.01171875f);  // 6/512: an all-zero group keeps a nonzero scale
        const uint32_t sc = encode_e4m3(__fdiv_rn(m, 6.0f));
        s = stored = __builtin_amdgcn_cvt_pk_f32_fp8(sc, false)[0];
    } else {
        m = gomax(m, u2f(0x01C00000u));  // float32(6·2^-126) = 1.5·2^-124
        s = pow2ceil(m * (float)(1.0 / 6));
        stored = e8m0((f2u(s) >> 23) & 0xffu);  // the scale byte, as DequantFP4 reads it
    }
    const uint32_t c = encode_e2m1(gomin(gomax(__fdiv_rn(v, s), -6.0f), 6.0f));
    const float grid[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};  // mx.go:45 fp4Grid
    const float fv = (c & 8) ? -grid[c & 7] : grid[c & 7];
    if (in) x[i] = round_bf16(fv * stored);
}

// E bytes a lane loads per row (16, 8 or 4): buffer loads, so that a row
// past the matrix's end reads zeros (the hardware's range check) and the
// row's offset is a scalar added to the lane's fixed offset.
typedef int rk_v2i __attribute__((ext_vector_type(2)));
template <int E>
struct Chunk;
template <>
struct Chunk<16> {
    typedef rk_v4i T;
    static __device__ T load(__amdgpu_buffer_rsrc_t r, int v, int s) {
        return __builtin_amdgcn_raw_buffer_load_b128(r, v, s, kAuxStream);
    }
    static __device__ uint32_t word(const T &v, int k) { return (uint32_t)v[k]; }
};
template <>
struct Chunk<8> {
    typedef rk_v2i T;
    static __device__ T load(__amdgpu_buffer_rsrc_t r, int v, int s) {
        return __builtin_amdgcn_raw_buffer_load_b64(r, v, s, kAuxStream);
    }
    static __device__ uint32_t word(const T &v, int k) { return (uint32_t)v[k]; }
};
template <>
struct Chunk<4> {
    typedef int T;
    static __device__ T load(__amdgpu_buffer_rsrc_t r, int v, int s) {
        return __builtin_amdgcn_raw_buffer_load_b32(r, v, s, kAuxStream);
    }
    static __device__ uint32_t word(const T &v, int) { return (uint32_t)v; }
};

// Row steps a workgroup loads at once (every lane holds RT weight chunks in
// registers; the fastest measured on MI355X, from 4 to 16 and with a
// persistent double-buffered variant, which was slower). For E4M3, RT
// divides 32: a tile's rows then share one row of 32x32-block scales.
constexpr int kMxStepsFp8 = 8;
constexpr int kMxStepsFp4 = 8;

// Terms per row in LDS: the row's blocks, padded to keep rows 16-byte
// aligned and spread over the banks.
__device__ __host__ constexpr int term_stride(int nb) { return ((nb + 3) & ~3) + 4; }

// Selected experts (internal/gpu/dsbatch.go:142-172 ExpertMatVecs): slot y
// of the launch multiplies expert ids[y] - e0 (if below experts) of S.per
// rows by input y / div into out + y·out_stride. ids null: one product.
struct MxSlots {
    const uint32_t *ids;
    int64_t per, out_stride;
    int32_t e0, experts, div;
};

// The lane's input slice, converted once: float64 values (E4M3 weights),
// or float16 pairs with the NaN codes' positions (E2M1 weights).
template <bool FP4, int NE>
struct XSlice;
template <int NE>
struct XSlice<false, NE> {
    double v[NE];
    __device__ void init(const uint32_t (&xw)[NE / 4]) {
#pragma unroll
        for (int k = 0; k < NE / 4; k++) {
            const rk_f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(xw[k], false);
            const rk_f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(xw[k], true);
            v[4 * k] = lo.x, v[4 * k + 1] = lo.y, v[4 * k + 2] = hi.x, v[4 * k + 3] = hi.y;
        }
    }
};
template <int NE>
struct XSlice<true, NE> {
    rk_h2 h[NE / 2];
    uint32_t nanmask;
    __device__ void init(const uint32_t (&xw)[NE / 4]) {
        nanmask = 0;
#pragma unroll
        for (int k = 0; k < NE / 4; k++) {
            uint32_t u = xw[k];
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (((u >> (8 * j)) & 0x7f) == 0x7f) {  // NaN code: 0 here, its position kept
                    nanmask |= 1u << (4 * k + j);
                    u &= ~(0xffu << (8 * j));
                }
            h[2 * k] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u, 1.0f, false);
            h[2 * k + 1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u, 1.0f, true);
        }
    }
};

// Where a lane's loads go: G rows side by side, each lane one block of row
// gl of each step.
struct MxLane {
    __amdgpu_buffer_rsrc_t rw, rsc;
    int vo;       // the lane's byte offset in a step
    int gl, b, nb, G;
    int64_t rb;   // weight bytes a row
};

// Tile t's loads: RT steps, step r taking row g·RT + r of the tile for each
// of the G rows side by side (weights, then scale bytes), issued
// unconditionally; rows past the part read zeros (buffer range check).
template <bool FP4, bool SIDE, int LB, int RT, typename WT>
__device__ __forceinline__ void mx_load_tile(const MxLane &L, int64_t t, WT (&wv)[RT], uint32_t (&wsv)[RT]) {
    typedef Chunk<FP4 ? 16 / LB : 32 / LB> WC;
    const int64_t row0 = t * RT * L.G;
#pragma unroll
    for (int r = 0; r < RT; r++) wv[r] = WC::load(L.rw, L.vo, (int)((row0 + r) * L.rb));
    if constexpr (FP4) {
        // the lane's RT rows' scale bytes, stored together (blocks of RT rows)
        const typename Chunk<RT>::T sb = Chunk<RT>::load(L.rsc, (L.gl * L.nb + L.b) * RT, (int)(row0 * L.nb));
#pragma unroll
        for (int r = 0; r < RT; r++) wsv[r] = (Chunk<RT>::word(sb, r >> 2) >> (8 * (r & 3))) & 0xffu;
    } else if constexpr (!SIDE) {
        // RT divides 32: the tile's rows share one row of 32x32-block scales
        const uint32_t s1 = __builtin_amdgcn_raw_buffer_load_b8(L.rsc, L.b, (int)((row0 >> 5) * L.nb), 0);
#pragma unroll
        for (int r = 0; r < RT; r++) wsv[r] = s1;
    } else {
        // the lane's RT rows are consecutive from a multiple of RT (which
        // divides 32): one row of 32x32-block scales too
        const uint32_t s1 =
            __builtin_amdgcn_raw_buffer_load_b8(L.rsc, (int)((row0 + L.gl * RT) >> 5) * L.nb + L.b, 0, 0);
#pragma unroll
        for (int r = 0; r < RT; r++) wsv[r] = s1;
    }
}

// One tile's terms into LDS, terms[(g·RT + r)·ts + block]: the exact block
// sums, combined over the block's LB lanes, rounded to float32, times the
// input's scale, times the weight's.
template <bool FP4, int LB, int RT, typename WT>
__device__ __forceinline__ void mx_tile_terms(const WT (&wv)[RT], const uint32_t (&wsv)[RT],
                                              const XSlice<FP4, 32 / LB> &x, float xsb, bool write, int G, int g,
                                              int bi, int ts, float *terms) {
    constexpr int NE = 32 / LB;
    constexpr int WB = FP4 ? NE / 2 : NE;
    typedef Chunk<WB> WC;
#pragma unroll
    for (int r = 0; r < RT; r++) {
        float t;
        if constexpr (!FP4) {
            double s0 = 0.0, s1 = 0.0;
#pragma unroll
            for (int k = 0; k < NE / 4; k++) {
                const uint32_t u = WC::word(wv[r], k);
                const rk_f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(u, false);
                const rk_f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(u, true);
                s0 = __builtin_fma((double)lo.x, x.v[4 * k], s0);
                s1 = __builtin_fma((double)lo.y, x.v[4 * k + 1], s1);
                s0 = __builtin_fma((double)hi.x, x.v[4 * k + 2], s0);
                s1 = __builtin_fma((double)hi.y, x.v[4 * k + 3], s1);
            }
            double d = s0 + s1;  // exact: every partial sum is
#pragma unroll
            for (int o = 1; o < LB; o <<= 1) d += __shfl_xor(d, o);
            t = (float)d;
        } else {
            uint32_t isum = 0;
#pragma unroll
            for (int k = 0; k < WB / 4; k++) {
                const uint32_t u = WC::word(wv[r], k);  // 8 weights
                const rk_h2 w0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1024.0f, 0);
                const rk_h2 w1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1024.0f, 1);
                const rk_h2 w2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1024.0f, 2);
                const rk_h2 w3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(u, 1024.0f, 3);
                const float f0 =
                    __builtin_amdgcn_fdot2(w1, x.h[4 * k + 1], __builtin_amdgcn_fdot2(w0, x.h[4 * k], 0.0f, false), false);
                const float f1 =
                    __builtin_amdgcn_fdot2(w3, x.h[4 * k + 3], __builtin_amdgcn_fdot2(w2, x.h[4 * k + 2], 0.0f, false), false);
                isum += (uint32_t)(int32_t)f0 + (uint32_t)(int32_t)f1;
            }
            if (x.nanmask) {  // rare: an infinite or NaN input in the block
                uint32_t odd = 0;
#pragma unroll
                for (int i = 0; i < NE; i++) {
                    const uint32_t nib = (WC::word(wv[r], i >> 3) >> (4 * (i & 7))) & 15u;
                    odd ^= ((x.nanmask >> i) & 1u) & (((nib & 5u) == 1u) ? 1u : 0u);
                }
                isum += odd << 31;
            }
#pragma unroll
            for (int o = 1; o < LB; o <<= 1) isum += (uint32_t)__shfl_xor((int)isum, o);
            t = (float)(int32_t)isum * 0.0009765625f;  // float32(sum / 1024): one rounding
        }
        if (write) {
            t = t * xsb;
            t = t * e8m0(wsv[r]);
            terms[(g * RT + r) * ts + bi] = t;
        }
    }
}

template <bool FP4, int LB>
__device__ __forceinline__ MxLane mx_lane(const uint8_t *w, const uint8_t *ws, int64_t rows, int nb, int G, int RT,
                                          int g, bool live, int b, int p) {
    constexpr int NE = 32 / LB, WB = FP4 ? NE / 2 : NE;
    MxLane L;
    L.rb = FP4 ? (int64_t)nb * 16 : (int64_t)nb * 32;
    // the part's weights and scales (under 2^31 bytes: launches are split)
    L.rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w), 0, (int)(rows * L.rb), kRsrcWord3);
    L.rsc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(ws), 0,
                                              (int)(FP4 ? (rows + RT - 1) / RT * RT * nb : (rows + 31) / 32 * nb),
                                              kRsrcWord3);
    L.gl = live ? g : 0;
    L.b = b;
    L.nb = nb;
    L.G = G;
    L.vo = L.gl * RT * (int)L.rb + b * (FP4 ? 16 : 32) + p * WB;
    return L;
}

// A workgroup takes RT·G rows: G runs of RT consecutive rows side by side
// (a step reads G rows at once; rows are contiguous, so a narrow matrix's
// rows read as long runs), RT steps. Lane group lg (LB lanes) takes block lg mod nb of row lg / nb
// within the step; rows wider than the workgroup's lanes take chunks of cb
// blocks (G = 1), the chains carried across them.
template <bool FP4, bool SIDE, int LB, int RT>
__global__ __launch_bounds__(512) void mx_matvec_kernel(const uint8_t *__restrict__ w, const uint8_t *__restrict__ ws,
                                                        int64_t rows, int cols, int G, const uint8_t *__restrict__ xc,
                                                        const float *__restrict__ xs, float *__restrict__ out,
                                                        int raw, MxSlots S) {
    if (S.ids) {
        // slot blockIdx.y: the expert its id names (rows experts of S.per
        // rows from w), its input, its output; ids outside the part are
        // another launch's (uniform per workgroup)
        const uint32_t e = S.ids[blockIdx.y] - (uint32_t)S.e0;
        if (e >= (uint32_t)S.experts) return;
        const int64_t nb = cols >> 5;
        w += (int64_t)e * S.per * (FP4 ? cols / 2 : cols);
        ws += FP4 ? (int64_t)e * S.per * nb : (int64_t)e * S.per / 32 * nb;
        rows = S.per;
        const int inp = blockIdx.y / S.div;
        xc += (int64_t)inp * cols;
        xs += (int64_t)inp * nb;
        out += blockIdx.y * S.out_stride;
    }
    constexpr int NE = 32 / LB;
    typedef typename Chunk<FP4 ? NE / 2 : NE>::T WT;
    extern __shared__ __align__(16) float terms[];
    const int tid = threadIdx.x, p = tid % LB, lg = tid / LB;
    const int nb = cols >> 5;
    const int groups = blockDim.x / LB;           // lane groups
    const int cb = SIDE ? nb : groups;            // blocks of a row per chunk
    const int g = SIDE ? lg / nb : 0;             // row within the step
    const bool live = SIDE ? g < G : true;        // idle groups past G·nb
    const int ts = term_stride(SIDE ? nb : cb);
    const int64_t row0 = (int64_t)blockIdx.x * RT * G;
    float acc = 0.0f;  // chain of row row0 + tid (tid < RT, G = 1)
    for (int c0 = 0; c0 < nb; c0 += cb) {  // uniform (one pass when SIDE)
        const int bi = SIDE ? lg % nb : lg;
        const int b = min(c0 + bi, nb - 1);  // past the last block: repeat it (its terms are not added)
        const MxLane L = mx_lane<FP4, LB>(w, ws, rows, nb, G, RT, g, live, b, p);
        // the input slice first (loads complete in issue order: it is then
        // ready while the weights are still on their way)
        uint32_t xw[NE / 4];
#pragma unroll
        for (int k = 0; k < NE / 4; k++) xw[k] = *reinterpret_cast<const uint32_t *>(xc + b * 32 + p * NE + 4 * k);
        const float xsb = xs[b];
        WT wv[RT];
        uint32_t wsv[RT];
        mx_load_tile<FP4, SIDE, LB, RT>(L, blockIdx.x, wv, wsv);
        XSlice<FP4, NE> x;
        x.init(xw);
        mx_tile_terms<FP4, LB, RT>(wv, wsv, x, xsb, p == 0 && live, G, g, bi, ts, terms);
        __syncthreads();
        if constexpr (SIDE) {
            // one chunk: every row's chain at once, rows strided over the threads
            for (int rl = tid; rl < RT * G; rl += blockDim.x) {
                if (row0 + rl >= rows) break;
                const float v = canonical(lds_chain_sum(terms + rl * ts, nb, 0.0f));
                out[row0 + rl] = raw ? v : round_bf16(v);
            }
            return;
        }
        if (tid < RT) acc = lds_chain_sum(terms + tid * ts, min(cb, nb - c0), acc);
        __syncthreads();  // the terms are read before the next chunk writes them
    }
    if (tid < RT && row0 + tid < rows) {
        const float v = canonical(acc);
        out[row0 + tid] = raw ? v : round_bf16(v);
    }
}

// Launch shape for nb blocks a row: lanes per block LB (the widest load
// first: 16 bytes), rows side by side G and waves W, for the fewest idle
// lanes; rows wider than 8 waves' lanes take chunks (G = 1).
struct MxShape {
    int lb, g, waves;
};
// Launch shapes measured faster on MI355X than the rule below picks, for
// DeepSeek-V4.1's widths: {E2M1?, blocks a row, rows side by side, waves}.
struct MxTune {
    bool fp4;
    int nb, g, waves;
};
constexpr MxTune kMxTune[] = {
    {true, 160, 1, 3},  // 5120 columns: 13824x5120 11.8 us against 14.3 (G = 2, 5 waves)
    {true, 72, 3, 4},   // 2304 columns: 5120x2304 5.4 us against 6.4 (G = 7, 8 waves)
};

MxShape mx_shape(bool fp4, int nb) {
    const int lb = fp4 ? 1 : 2;  // 16-byte loads
    for (const MxTune &t : kMxTune)
        if (t.fp4 == fp4 && t.nb == nb) return MxShape{lb, t.g, t.waves};
    const int64_t lanes = (int64_t)nb * lb;
    MxShape best{lb, 1, 8};
    int64_t best_key = -1;
    for (int W = 1; W <= 8; W++) {
        const int64_t per = 64 * W;
        int64_t G = std::min<int64_t>(per / lanes, 16), waste, chunks = 1;
        if (G >= 1) {
            waste = per - G * lanes;
        } else {
            G = 1;
            chunks = (lanes + per - 1) / per;
            waste = chunks * per - lanes;
        }
        if (waste >= 64) continue;  // a whole idle wave
        // the fewest idle lanes, then the fewest chunks, then the most
        // rows side by side
        const int64_t key = waste * 65536 + chunks * 256 + (16 - G);  // G <= 16
        if (best_key < 0 || key < best_key) {
            best_key = key;
            best = MxShape{lb, (int)G, W};
        }
    }
    return best;
}

template <bool FP4, bool SIDE, int LB, int RT>
void launch_mx_t(const uint8_t *w, const uint8_t *ws, int64_t rows, int cols, const uint8_t *xc, const float *xs,
                 float *out, bool raw, int G, int waves, const MxSlots &S, int slots, hipStream_t s) {
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute((const void *)mx_matvec_kernel<FP4, SIDE, LB, RT>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    const int nb = cols / 32, cb = SIDE ? nb : 64 * waves / LB;
    const size_t lds = (size_t)RT * G * term_stride(cb) * 4;
    const int64_t per = (int64_t)RT * G;
    const int64_t tiles = (rows + per - 1) / per;
    RK_LAUNCH((mx_matvec_kernel<FP4, SIDE, LB, RT>), dim3((unsigned)tiles, (unsigned)slots), dim3((unsigned)(64 * waves)),
              lds, s, w, ws, rows, cols, G, xc, xs, out, raw ? 1 : 0, S);
}

void launch_mx_any(bool fp4, const MxShape &sh, const uint8_t *w, const uint8_t *ws, int64_t rows, int cols,
                   const uint8_t *xc, const float *xs, float *out, bool raw, const MxSlots &S, int slots,
                   hipStream_t s) {
    if (fp4 && sh.g > 1)
        launch_mx_t<true, true, 1, kMxStepsFp4>(w, ws, rows, cols, xc, xs, out, raw, sh.g, sh.waves, S, slots, s);
    else if (fp4)
        launch_mx_t<true, false, 1, kMxStepsFp4>(w, ws, rows, cols, xc, xs, out, raw, 1, sh.waves, S, slots, s);
    else if (sh.g > 1)
        launch_mx_t<false, true, 2, kMxStepsFp8>(w, ws, rows, cols, xc, xs, out, raw, sh.g, sh.waves, S, slots, s);
    else
        launch_mx_t<false, false, 2, kMxStepsFp8>(w, ws, rows, cols, xc, xs, out, raw, 1, sh.waves, S, slots, s);
}

}  // namespace

int64_t mx_fp4_scale_bytes(int64_t rows, int64_t cols) {
    return (rows + kMxStepsFp4 - 1) / kMxStepsFp4 * kMxStepsFp4 * (cols / 32);
}

void mx_fp4_pack_scales(const uint8_t *e8m0, int64_t rows, int64_t cols, uint8_t *dst) {
    const int64_t RT = kMxStepsFp4, nb = cols / 32, total = mx_fp4_scale_bytes(rows, cols);
    for (int64_t i = 0; i < total; i++) {
        // i = (k·nb + b)·RT + r holds row k·RT + r, block b
        const int64_t r = i % RT, b = (i / RT) % nb, row = i / (RT * nb) * RT + r;
        dst[i] = row < rows ? e8m0[row * nb + b] : 0;
    }
}

void launch_act_fp8(const float *x, int64_t n, uint8_t *codes, float *scales, hipStream_t s) {
    if (n <= 0) return;
    RK_LAUNCH(act_fp8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n, codes, scales);
}

void launch_e4m3_values(const uint8_t *codes, int64_t n, float *out, hipStream_t s) {
    if (n <= 0) return;
    RK_LAUNCH(e4m3_values_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, codes, n, out);
}

void launch_act_quant_inplace(float *x, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    RK_LAUNCH(act_quant_inplace_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n);
}

void launch_fp4_quant_inplace(float *x, int64_t n, bool e4m3, hipStream_t s) {
    if (n <= 0) return;
    if (e4m3)
        RK_LAUNCH(fp4_quant_inplace_kernel<true>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n);
    else
        RK_LAUNCH(fp4_quant_inplace_kernel<false>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n);
}

void launch_mx_matvec(bool fp4, const uint8_t *w, const uint8_t *ws, int64_t rows, int64_t cols, const uint8_t *xc,
                      const float *xs, float *out, bool raw, hipStream_t s) {
    const MxShape sh = mx_shape(fp4, (int)(cols / 32));
    const int64_t rb = fp4 ? cols / 2 : cols, nb = cols / 32;
    // parts of at most 1 GiB of weights, whole 32-row scale blocks (and so
    // whole blocks of the E2M1 scales' RT rows)
    const int64_t align = 32;
    const int64_t per = std::max<int64_t>(align, ((int64_t)1 << 30) / rb / align * align);
    const MxSlots none{nullptr, 0, 0, 0, 0, 1};
    for (int64_t r0 = 0; r0 < rows; r0 += per) {
        const int64_t n = std::min(per, rows - r0);
        launch_mx_any(fp4, sh, w + r0 * rb, ws + (fp4 ? r0 * nb : r0 / 32 * nb), n, (int)cols, xc, xs, out + r0, raw,
                      none, 1, s);
    }
}

void launch_mx_experts(const uint8_t *w, const uint8_t *ws, int64_t experts, int64_t per_expert, int64_t cols,
                       const uint32_t *ids, int slots, int div, const uint8_t *xc, const float *xs, float *out,
                       int64_t out_stride, bool raw, hipStream_t s) {
    const MxShape sh = mx_shape(true, (int)(cols / 32));
    const int64_t rb = cols / 2, nb = cols / 32;
    // parts of whole experts, at most 1 GiB of weights each
    const int64_t per = std::max<int64_t>(1, ((int64_t)1 << 30) / rb / per_expert);
    for (int64_t e0 = 0; e0 < experts; e0 += per) {
        const int64_t ne = std::min(per, experts - e0);
        const MxSlots S{ids, per_expert, out_stride, (int32_t)e0, (int32_t)ne, div};
        launch_mx_any(true, sh, w + e0 * per_expert * rb, ws + e0 * per_expert * nb, per_expert, (int)cols, xc, xs, out,
                      raw, S, slots, s);
    }
}

}  // namespace rk
