// rk_dev.h — device helpers shared by the gfx950 kernels: wave-level
// integer dot products and reductions, the Dot32 summation order, the
// activation quantizer of one 4-element group, and streaming loads.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rk_fmath.h"

namespace rk {

// 16-byte load marked non-temporal: weights are streamed once per product,
// so they should not displace the activations kept in the caches.
typedef int rk_v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 load_stream16(const void *p) {
    const rk_v4i v = __builtin_nontemporal_load(reinterpret_cast<const rk_v4i *>(p));
    return make_int4(v.x, v.y, v.z, v.w);
}

// Loads through a pointer known to be global memory. A pointer read from
// memory (a table of per-expert rows) is generic to the compiler, which then
// issues flat loads; those count against the LDS wait counter too, so every
// wait for an LDS access would also wait for them.
typedef const __attribute__((address_space(1))) rk_v4i *rk_gv4i;
typedef const __attribute__((address_space(1))) float *rk_gf;
__device__ __forceinline__ int4 load_stream16_g(const void *p) {
    const rk_v4i v = __builtin_nontemporal_load((rk_gv4i)p);
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ int4 load16_g(const void *p) {
    const rk_v4i v = *(rk_gv4i)p;
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float loadf_g(const float *p) { return *(rk_gf)p; }

// Exact integer sum of a lane pair (quad_perm [1,0,3,2]).
__device__ __forceinline__ int pair_sum(int s) { return s + __builtin_amdgcn_mov_dpp(s, 0xB1, 0xF, 0xF, false); }

// acc + Σ w_j·x_j over 16 signed bytes (four v_dot4_i32_i8), exact.
__device__ __forceinline__ int dot16(int4 w, int4 x, int acc) {
    acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
    acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
    acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
    acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
    return acc;
}

// Dot32 (internal/num/matvec.go:32-66) by the 32 lanes of a half-wave
// (`hl` = lane in the half): element i goes into running sum i mod 32, in
// order of i; then e_j = (s_j + s_j+8) + (s_j+16 + s_j+24) and the tree
// ((e0+e1)+(e2+e3))+((e4+e5)+(e6+e7)). The result is valid in the half's
// lane 0. Every lane of the wave must call it (cross-lane moves).
__device__ __forceinline__ float dot32_reduce(float s) {
    const float s8 = __shfl_down(s, 8, 32), s16 = __shfl_down(s, 16, 32), s24 = __shfl_down(s, 24, 32);
    const float e = (s + s8) + (s16 + s24);
    const float p = e + __shfl_down(e, 1, 32);
    const float q = p + __shfl_down(p, 2, 32);
    return q + __shfl_down(q, 4, 32);
}

__device__ __forceinline__ float dot32_half(const float *a, const float *b, int n, int hl, bool valid) {
    float s = 0.0f;
    if (valid)
        for (int i = hl; i < n; i += 32) s += a[i] * b[i];
    return dot32_reduce(s);
}

// acc + p[0] + ... + p[N-1] in order (float32), p in LDS, 16-byte aligned:
// straight-line code, so the compiler issues the reads (immediate offsets
// from one address) well ahead of the additions that wait on them.
template <int N>
__device__ __forceinline__ float lds_sum_fixed(const float *p, float acc) {
    const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int k = 0; k < N / 4; k++) {
        const float4 v = q[k];
        acc += v.x;
        acc += v.y;
        acc += v.z;
        acc += v.w;
    }
    return acc;
}

// Buffer descriptor word 3 of an untyped 32-bit raw buffer (gfx9 family),
// and the cache policy of a streamed weight load (non-temporal).
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kAuxStream = 2;
// The cache policy of an agent-scope load (sc1: the level where every XCD
// sees the same data), as the compiler gives a relaxed agent-scope atomic
// load.
constexpr int kAuxCoherent = 16;

// The LDS address space form of a pointer into the kernel's LDS (the
// destination operand of a direct-to-LDS load).
__device__ __forceinline__ __attribute__((address_space(3))) void *lds_ptr(void *p) {
    return (__attribute__((address_space(3))) void *)p;
}

// s_waitcnt operand (gfx9) waiting for vector memory operations until at
// most n remain outstanding, and for nothing else.
constexpr int vmcnt_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Software pipeline of a sequential LDS sum: batches of kChainBatch float4,
// the next batch's reads issued before the current batch's additions. The
// scheduling barriers keep the compiler from sinking the reads next to their
// uses (it otherwise keeps one read in flight to save registers, and every
// four additions then wait out a whole LDS latency).
constexpr int kChainBatch = 8;

__device__ __forceinline__ void lds_load_batch(float4 (&b)[kChainBatch], const float4 *q) {
#pragma unroll
    for (int k = 0; k < kChainBatch; k++) b[k] = q[k];
}

__device__ __forceinline__ float add_batch(const float4 (&b)[kChainBatch], float acc) {
#pragma unroll
    for (int k = 0; k < kChainBatch; k++) {
        acc += b[k].x;
        acc += b[k].y;
        acc += b[k].z;
        acc += b[k].w;
    }
    return acc;
}

// acc + p[0] + p[1] + ... + p[n-1], added one at a time in order (float32),
// from LDS (p 16-byte aligned).
__device__ __forceinline__ float lds_chain_sum(const float *p, int n, float acc) {
    constexpr int kPer = 4 * kChainBatch;  // floats per batch
    const float4 *q = reinterpret_cast<const float4 *>(p);
    const int nb = n / kPer;
    if (nb > 0) {
        float4 a[kChainBatch], b[kChainBatch];
        lds_load_batch(a, q);
        int k = 1;
        for (; k + 1 < nb; k += 2) {
            lds_load_batch(b, q + k * kChainBatch);
            __builtin_amdgcn_sched_barrier(0);
            acc = add_batch(a, acc);
            __builtin_amdgcn_sched_barrier(0);
            lds_load_batch(a, q + (k + 1) * kChainBatch);
            __builtin_amdgcn_sched_barrier(0);
            acc = add_batch(b, acc);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (k < nb) {
            lds_load_batch(b, q + k * kChainBatch);
            __builtin_amdgcn_sched_barrier(0);
            acc = add_batch(a, acc);
            __builtin_amdgcn_sched_barrier(0);
            acc = add_batch(b, acc);
        } else {
            acc = add_batch(a, acc);
        }
    }
    int t = nb * kPer;
    for (; t + 16 <= n; t += 16) acc = lds_sum_fixed<16>(p + t, acc);
    for (; t < n; t++) acc += p[t];
    return acc;
}

// Dot32's running sum of lane j (< 32) for x·x: x_i·x_i for i = j, j+32,
// ... in order, from LDS holding x transposed (xt[j·pitch + m] = x_{j+32m},
// pitch a multiple of 4, m < steps), in fixed-size straight-line pieces.
template <int N>
__device__ __forceinline__ float lds_sq_fixed(const float *p, float s) {
    const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int k = 0; k < N / 4; k++) {
        const float4 v = q[k];
        s += v.x * v.x;
        s += v.y * v.y;
        s += v.z * v.z;
        s += v.w * v.w;
    }
    return s;
}

__device__ __forceinline__ float lds_dot32_self_t(const float *xt, int pitch, int steps, int j) {
    const float *row = xt + j * pitch;
    float s = 0.0f;
    int m = 0;
    for (; m + 64 <= steps; m += 64) s = lds_sq_fixed<64>(row + m, s);
    for (; m + 16 <= steps; m += 16) s = lds_sq_fixed<16>(row + m, s);
    for (; m < steps; m++) s += row[m] * row[m];
    return s;
}

// Lane exchanges inside aligned groups of eight lanes, by DPP (no LDS
// round trip): xor 1 and xor 2 are quad permutations, and the half-row
// mirror (lane i <-> 7-i) pairs each quad with the other. Applied in that
// order with an associative, commutative operation, every lane of the eight
// ends with the result over all eight.
__device__ __forceinline__ int dpp_x1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int dpp_x2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false); }
__device__ __forceinline__ int dpp_mirror8(int v) { return __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false); }

__device__ __forceinline__ float dppf_x1(float v) { return __int_as_float(dpp_x1(__float_as_int(v))); }
__device__ __forceinline__ float dppf_x2(float v) { return __int_as_float(dpp_x2(__float_as_int(v))); }

// Go max inside each row of 16 lanes, valid in every lane of the row: DPP
// xor 1, xor 2, half-row mirror, row mirror. Go max (NaN wins, +0 over -0)
// is associative and commutative, so the order is free.
__device__ __forceinline__ float row16_gomax(float m) {
    m = gomax(m, dppf_x1(m));
    m = gomax(m, dppf_x2(m));
    m = gomax(m, __int_as_float(dpp_mirror8(__float_as_int(m))));
    return gomax(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x140, 0xF, 0xF, false)));
}

// Go max over each half-wave (lanes 0-31, 32-63), valid in every lane of
// the half. Every lane of the wave must call it.
__device__ __forceinline__ float half_gomax(float m) {
    m = row16_gomax(m);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 48));
    return (threadIdx.x & 32) ? gomax(r2, r3) : gomax(r0, r1);
}

// Go max over the wave, valid in every lane: the rows, then the four rows by
// readlane. Every lane of the wave must call it.
__device__ __forceinline__ float wave_gomax(float m) {
    m = row16_gomax(m);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 48));
    return gomax(gomax(r0, r1), gomax(r2, r3));
}

// Q8_0 activation quantizer (internal/num/quant.go:34-53) of one group of
// four values, eight lanes (aligned) per 32-value block: returns the four
// codes packed little-endian, and the block's scale and code sum (valid in
// every lane of the eight). Every lane of the wave must call it. The block
// maximum (Go max: NaN wins, +0 over -0) and the integer sum are exact in
// any order.
__device__ __forceinline__ uint32_t quantize_group(float v0, float v1, float v2, float v3, float &d, int &csum) {
    float a = abs_max3(abs_max3(0.0f, v0, v1), v2, v3);
    a = __builtin_elementwise_maximum(a, dppf_x1(a));
    a = __builtin_elementwise_maximum(a, dppf_x2(a));
    a = __builtin_elementwise_maximum(a, __int_as_float(dpp_mirror8(__float_as_int(a))));
    a = canonical(a);  // Go max gives the canonical NaN
    d = a * u2f(k1_127);
    // a zero or NaN scale gives codes 0 (quant.go:44-46): v·0 is ±0 or NaN,
    // both code 0, so the codes need no branch
    const bool zero = (d == 0.0f) || (d != d);
    const float id = zero ? 0.0f : recip32(d);
    const int c0 = q8_code(v0, id), c1 = q8_code(v1, id), c2 = q8_code(v2, id), c3 = q8_code(v3, id);
    int s = c0 + c1 + c2 + c3;
    s += dpp_x1(s);
    s += dpp_x2(s);
    s += dpp_mirror8(s);
    csum = s;
    return (uint32_t)(c0 & 255) | ((uint32_t)(c1 & 255) << 8) | ((uint32_t)(c2 & 255) << 16) |
           ((uint32_t)(c3 & 255) << 24);
}

// Q8_0 quantization (internal/num/quant.go:34-53) of one 32-value block
// held by one lane: Recip32 once per block. Codes packed little-endian four
// to a word; the block's scale and code sum.
__device__ __forceinline__ void quantize_block32(const float4 (&v)[8], uint32_t (&pk)[8], float &d, int &csum) {
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) a = abs_max3(abs_max3(a, v[k].x, v[k].y), v[k].z, v[k].w);
    a = canonical(a);
    d = a * u2f(k1_127);
    // a zero or NaN scale gives codes 0 (v·0 is ±0 or NaN: code 0, no branch)
    const bool zero = (d == 0.0f) || (d != d);
    const float id = zero ? 0.0f : recip32(d);
    int s = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int c0 = q8_code(v[k].x, id), c1 = q8_code(v[k].y, id), c2 = q8_code(v[k].z, id), c3 = q8_code(v[k].w, id);
        s += (c0 + c1) + (c2 + c3);
        pk[k] = (uint32_t)(c0 & 255) | ((uint32_t)(c1 & 255) << 8) | ((uint32_t)(c2 & 255) << 16) |
                ((uint32_t)(c3 & 255) << 24);
    }
    csum = s;
}

// a = silu(v)·b (internal/llm/model.go:657, :603-605).
__device__ __forceinline__ float silu_mul(float v, float b) {
    const float sl = v * recip32(1.0f + exp32(-v));
    return sl * b;
}

// Greedy-argmax merge (internal/llm/sample.go:45-53: the first index holding
// the largest value wins): candidate (v, i) replaces (bv, bi) if it is
// larger, or equal at a lower index. bi < 0 marks "none yet"; NaNs are never
// candidates.
__device__ __forceinline__ void argmax_merge(float &bv, int &bi, float v, int i) {
    if (i < 0) return;
    if (bi < 0 || v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// 64-bit key of logit v (not NaN) at row i for a max-reduction that picks
// the first row holding the largest value: the float's order-preserving
// bits above (-0 taken as +0, which compare equal), the complement of the
// row below. Never 0.
__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
    uint32_t u = f2u(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)i);
}

// ---- Row dots eight lanes a row: lane l of an aligned group of eight keeps
// MatVecQ8's running sum l (blocks l, l+8, ... in order, from +0) of one
// row, from the row's blocks it holds in registers; tree8 then forms
// ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7)) with no other lane exchange. ----

// The row's blocks rl + 8m, m < BPL (clamped into the row: those past it
// are never summed), row and rs in global memory. STREAM: non-temporal
// loads, for rows read once.
template <int BPL, bool STREAM = true>
__device__ __forceinline__ void lane_row_load(int4 (&c0)[BPL], int4 (&c1)[BPL], float (&sw)[BPL], const uint8_t *row,
                                              const float *rs, int nb, int rl) {
#pragma unroll
    for (int m = 0; m < BPL; m++) {
        const int b = min(rl + 8 * m, nb - 1);
        if (STREAM) {
            c0[m] = load_stream16_g(row + 32 * b);
            c1[m] = load_stream16_g(row + 32 * b + 16);
        } else {
            c0[m] = load16_g(row + 32 * b);
            c1[m] = load16_g(row + 32 * b + 16);
        }
        sw[m] = loadf_g(rs + b);
    }
}

// Running sum rl of the held row with one input (xq: codes, xsc: block
// scales), continued from acc: exact block sums, times (row scale · input
// scale), added in order.
template <int BPL>
__device__ __forceinline__ float lane_running_sum_from(float acc, const int4 (&c0)[BPL], const int4 (&c1)[BPL],
                                                       const float (&sw)[BPL], const int8_t *xq, const float *xsc,
                                                       int nb, int rl) {
#pragma unroll
    for (int m = 0; m < BPL; m++) {
        const int b = rl + 8 * m;
        if (b < nb) {
            const int4 *xp = reinterpret_cast<const int4 *>(xq + 32 * b);
            const int sum = dot16(c1[m], xp[1], dot16(c0[m], xp[0], 0));
            acc += (float)sum * (sw[m] * xsc[b]);
        }
    }
    return acc;
}

// The same from +0 (a row's blocks held whole).
template <int BPL>
__device__ __forceinline__ float lane_running_sum(const int4 (&c0)[BPL], const int4 (&c1)[BPL], const float (&sw)[BPL],
                                                  const int8_t *xq, const float *xsc, int nb, int rl) {
    return lane_running_sum_from<BPL>(0.0f, c0, c1, sw, xq, xsc, nb, rl);
}

// The fixed tree over the group's eight running sums, valid in all eight
// lanes (float addition commutes, so each lane's pairing gives the same bits).
__device__ __forceinline__ float tree8(float acc) {
    acc = acc + dppf_x1(acc);
    acc = acc + dppf_x2(acc);
    return acc + __int_as_float(dpp_mirror8(__float_as_int(acc)));
}

// ---- The same row dots with the row read in contiguous 16-byte pieces (a
// 128-byte line per load instruction and row): at step k (k < 2·BPL) lane
// rl holds half rl & 1 of block 4k + rl/2, so a lane pair holds a block.
// Lane 2p keeps running sum p (the even steps: blocks 8m + p) and lane
// 2p+1 running sum 4 + p (the odd steps: blocks 8m + 4 + p), each in block
// order from +0, the block's exact sum formed from the pair's two dots by
// one DPP exchange; tree8_pair forms the same tree. Measured on MI355X: 64
// rows a workgroup read about 15 % faster than as whole 32-byte blocks a
// lane. With the input offsets clamped (rows of any width) it holds more
// registers where a row is summed against several inputs; at rows of
// exactly 8·BPL blocks (EXACT) fewer. Kernels that would drop below four
// waves a SIMD keep the first form. ----

// The running sum a lane keeps (its m-th term is block L + 8m).
__device__ __forceinline__ int pair_sum_index(int rl) { return (rl & 1) ? 4 + (rl >> 1) : rl >> 1; }

// c0[m] at byte 256m + 16·rl, c1[m] at 256m + 128 + 16·rl (clamped into
// the row: what lies past it is never summed), and the scales of the
// lane's own blocks.
template <int BPL, bool STREAM = true>
__device__ __forceinline__ void lane_row_load_pair(int4 (&c0)[BPL], int4 (&c1)[BPL], float (&sw)[BPL],
                                                   const uint8_t *row, const float *rs, int nb, int rl) {
    const int last = 32 * nb - 16, L = pair_sum_index(rl);
#pragma unroll
    for (int m = 0; m < BPL; m++) {
        const int o0 = min(256 * m + 16 * rl, last), o1 = min(256 * m + 128 + 16 * rl, last);
        if (STREAM) {
            c0[m] = load_stream16_g(row + o0);
            c1[m] = load_stream16_g(row + o1);
        } else {
            c0[m] = load16_g(row + o0);
            c1[m] = load16_g(row + o1);
        }
        sw[m] = loadf_g(rs + min(L + 8 * m, nb - 1));
    }
}

// The lane's running sum of the row held by lane_row_load_pair with one
// input, continued from acc. Every lane of the group calls it. EXACT: the
// row is exactly 8·BPL blocks (nb is not read), so the input's offsets
// need no clamp and fold into the reads' immediate offsets.
template <int BPL, bool EXACT = false>
__device__ __forceinline__ float lane_running_sum_pair_from(float acc, const int4 (&c0)[BPL], const int4 (&c1)[BPL],
                                                            const float (&sw)[BPL], const int8_t *xq, const float *xsc,
                                                            int nb, int rl) {
    const int last = 32 * nb - 16, L = pair_sum_index(rl);
    const bool odd = rl & 1;
#pragma unroll
    for (int m = 0; m < BPL; m++) {
        const int o0 = EXACT ? 256 * m + 16 * rl : min(256 * m + 16 * rl, last);
        const int o1 = EXACT ? 256 * m + 128 + 16 * rl : min(256 * m + 128 + 16 * rl, last);
        const int d0 = dot16(c0[m], *reinterpret_cast<const int4 *>(xq + o0), 0);
        const int d1 = dot16(c1[m], *reinterpret_cast<const int4 *>(xq + o1), 0);
        // the block this lane keeps: its own half's dot plus the partner's
        // (each lane sends the half its partner keeps)
        const int sum = (odd ? d1 : d0) + __builtin_amdgcn_mov_dpp(odd ? d0 : d1, 0xB1, 0xF, 0xF, false);
        const int b = L + 8 * m;
        if (EXACT || b < nb) acc += (float)sum * (sw[m] * xsc[b]);
    }
    return acc;
}

template <int BPL, bool EXACT = false>
__device__ __forceinline__ float lane_running_sum_pair(const int4 (&c0)[BPL], const int4 (&c1)[BPL],
                                                       const float (&sw)[BPL], const int8_t *xq, const float *xsc,
                                                       int nb, int rl) {
    return lane_running_sum_pair_from<BPL, EXACT>(0.0f, c0, c1, sw, xq, xsc, nb, rl);
}

// The tree over running sums held as lane_running_sum_pair leaves them
// (lane 2p: s_p, lane 2p+1: s_4+p): lanes 2 apart give s0+s1, s2+s3,
// s4+s5, s6+s7; lanes 4 apart (the half-row mirror, then the quad
// reversed) the two halves; then the lane pair. Valid in all eight lanes.
__device__ __forceinline__ float tree8_pair(float acc) {
    acc = acc + dppf_x2(acc);
    const int m8 = dpp_mirror8(__float_as_int(acc));
    acc = acc + __int_as_float(__builtin_amdgcn_mov_dpp(m8, 0x1B, 0xF, 0xF, false));
    return acc + dppf_x1(acc);
}

// RMSNorm (internal/llm/model.go:632-638: ss = Dot32(x,x)·recip_n + eps,
// out_i = w_i·(Rsqrt32(ss)·x_i)) of x, then the Q8_0 quantization
// (internal/num/quant.go:34-53) of the result into qx/xs/xsum: the input of
// the next product. Thread t holds groups g = t + k·NT (four values each)
// of x and w in registers, loaded before the call; sx is LDS for n floats.
// Every thread of the NT-thread workgroup calls it.
template <int NT, int MAXG>
__device__ void wg_norm_quant(const float4 *xv, const float4 *wv, int n, float recip_n, float eps, int8_t *qx,
                              float *xs, int32_t *xsum, float *sx, float *bcast) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int ng = n >> 2;
    // x transposed for Dot32: xt[j·pitch + m] = x_{j+32m} (n a multiple of 32)
    const int steps = n >> 5, pitch = ((steps + 3) & ~3) + 4;
#pragma unroll
    for (int k = 0; k < MAXG; k++) {
        const int g = tid + k * NT;
        if (g < ng) {
            const int i = 4 * g;
            float *d = sx + (i & 31) * pitch + (i >> 5);
            d[0] = xv[k].x;
            d[pitch] = xv[k].y;
            d[2 * pitch] = xv[k].z;
            d[3 * pitch] = xv[k].w;
        }
    }
    __syncthreads();
    if (tid < 64) {
        const float s = lane < 32 ? lds_dot32_self_t(sx, pitch, steps, lane) : 0.0f;
        const float dot = dot32_reduce(s);
        if (lane == 0) *bcast = rsqrt32((dot * recip_n) + eps);
    }
    __syncthreads();
    const float r = *bcast;
#pragma unroll
    for (int k = 0; k < MAXG; k++) {
        if (k * NT < ng) {  // uniform
            const int g = tid + k * NT;
            float d;
            int cs;
            const uint32_t pk = quantize_group(wv[k].x * (r * xv[k].x), wv[k].y * (r * xv[k].y),
                                               wv[k].z * (r * xv[k].z), wv[k].w * (r * xv[k].w), d, cs);
            if (g < ng) {
                reinterpret_cast<uint32_t *>(qx)[g] = pk;
                if ((g & 7) == 0) {
                    xs[g >> 3] = d;
                    xsum[g >> 3] = cs;
                }
            }
        }
    }
}

// LDS of wg_norm_quant for n values: x transposed, 32 rows of the pitch.
inline size_t norm_lds(int n) { return (size_t)32 * ((((n >> 5) + 3) & ~3) + 4) * 4; }


}  // namespace rk
