// rk_sample.hip — the generation step's choice of the next token, on the
// device: the greedy argmax of independent sequences, and the seeded
// sampler (internal/llm/sample.go:26-43) with its state on the device.
//
// Sampling a row of logits at temperature T (sample.go:30-41):
//   p_i = logit_i / T, softmax (model.go:640-654): mx = Go max of p,
//   e_i = Exp32(p_i - mx), S = e_0 + e_1 + ... in order (float32),
//   p'_i = e_i * Recip32(S); r = the xorshift64* draw; the token is the first
//   i with r < p'_0 + ... + p'_i (float32, in order), else the last index.
// Three launches: Go-max partials over many workgroups, the terms e_i into a
// buffer over many workgroups, then one workgroup a sequence for the two
// running sums and the draw.
//
// The running sums. A float32 running sum s_{k+1} = fl(s_k + t_k) of terms
// t_k >= 0 is a chain of dependent additions, ~150k of them for a vocabulary
// row. It is computed exactly in parallel instead: while s stays below the
// next power of two, every representable s is m·u for its ulp u and an
// integer m < 2^24, and adding t rounds to m' = m + rint(t/u) (t/u is exact:
// a power-of-two scaling), except when t/u is a tie (x.5: the even neighbour
// depends on m) or m' reaches 2^24 (the next binade's coarser grid). Between
// such events the sum is integer addition, which is associative: a
// workgroup scan over a chunk of terms (up to 8192) advances s at once. At an
// event the term is added as a float, the grid is re-read from the new s,
// and the chunk resumes after it. The first kSmpPre terms, where s is still
// small and events are dense, are added one by one.
#include "rk_dev.h"
#include "rk_fused.h"
#include "rk_runtime.h"

namespace rk {

namespace {

constexpr int kSmpThreads = 256;
constexpr int kSmpWaves = kSmpThreads / 64;
constexpr int kSmpPre = 256;                         // terms added one by one first
constexpr int kSmpParts = 256;                       // workgroups a row (max and terms)
constexpr int kSmpPartThreads = 256;
constexpr uint32_t kGridTop = 1u << 24;              // m reaches the next binade
constexpr uint32_t kGridCap = 1u << 25;              // saturation of the scans (past kGridTop)
constexpr int kNone = 0x7fffffff;

__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b) { return min(a + b, kGridCap); }

// s = m·2^eu for s >= 0 (not NaN): eu of s's binade (subnormals share the
// first normal binade's 2^-149), m < 2^24.
struct Grid {
    int eu;
    uint32_t m;
};

__device__ __forceinline__ Grid grid_of(float s) {
    const uint32_t b = f2u(s);
    const int e = (int)(b >> 23);
    return Grid{max(e, 1) - 150, e ? ((b & 0x7FFFFFu) | 0x800000u) : b};
}

// m·2^eu for m < 2^24 (m < 2^23 only on the subnormal grid, eu = -149).
__device__ __forceinline__ float grid_value(uint32_t m, int eu) {
    return m < 0x800000u ? u2f(m) : u2f(((uint32_t)(eu + 150) << 23) + (m - 0x800000u));
}

// Inclusive prefix sum over the wave's 64 lanes (sums below 2^32): within
// each row of 16 by row shifts, then across rows by the row broadcasts.
__device__ __forceinline__ uint32_t wave_scan_add(uint32_t v) {
    uint32_t t = v;
    t += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true);  // row_shr:1
    t += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true);  // row_shr:2
    t += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x113, 0xf, 0xf, true);  // row_shr:3
    t += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)t, 0x114, 0xf, 0xe, false); // row_shr:4, lanes 4-15
    t += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)t, 0x118, 0xf, 0xc, false); // row_shr:8, lanes 8-15
    t += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)t, 0x142, 0xa, 0xf, false); // row_bcast:15, rows 1, 3
    t += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)t, 0x143, 0xc, 0xf, false); // row_bcast:31, rows 2, 3
    return t;
}

struct SmpLds {
    uint32_t wt[kSmpWaves];  // the waves' sums
    int emin[2], hmin[2];    // a step's first event and first hit (r < running sum), by step parity
    float cand[kSmpThreads]; // each thread's running sum after its first event
    alignas(16) float pre[kSmpPre];
    float bv[kSmpWaves];
    int bi[kSmpWaves];
    int first;
    float r;
};

// p[i] <- p[0] + ... + p[i], added in order from +0 (float32), n a multiple
// of 32, in LDS; one lane.
__device__ void lds_chain_cum(float *p, int n) {
    float4 *q = reinterpret_cast<float4 *>(p);
    float acc = 0.0f;
    for (int b = 0; b < n / 4; b += kChainBatch) {
        float4 v[kChainBatch];
        lds_load_batch(v, q + b);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < kChainBatch; k++) {
            acc += v[k].x;
            v[k].x = acc;
            acc += v[k].y;
            v[k].y = acc;
            acc += v[k].z;
            v[k].z = acc;
            acc += v[k].w;
            v[k].w = acc;
        }
#pragma unroll
        for (int k = 0; k < kChainBatch; k++) q[b + k] = v[k];
    }
}

// One thread's terms on grid g for the positions [lo, hi) of its PER:
// running increments pre[] (from 0), and the events (a tie, or a term at or
// past the next binade, or NaN) as bits. Positions outside add nothing.
template <int PER, bool kChecked>
__device__ __forceinline__ uint32_t grid_terms(const float (&t)[PER], const Grid &g, int lo, int hi,
                                               uint32_t (&pre)[PER], uint32_t &evm) {
    uint32_t acc = 0;
    evm = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const float q = __builtin_amdgcn_ldexpf(t[j], -g.eu);
        const bool big = !(q < 16777216.0f);
        const float qs = big ? 0.0f : q;
        const float qr = __builtin_rintf(qs);
        const bool tie = __builtin_fabsf(qs - qr) == 0.5f;
        uint32_t inc = big ? kGridCap : (uint32_t)qr;
        bool ev = big || tie;
        if (kChecked) {
            const bool valid = j >= lo && j < hi;
            inc = valid ? inc : 0u;
            ev = ev && valid;
        }
        acc += inc;  // at most PER·2^25: no wrap
        pre[j] = acc;
        evm |= ev ? (1u << j) : 0u;
    }
    return acc;
}

// A chunk's terms for the thread: positions c0 + tid·PER + [0, PER), as
// float4 (c0 and the row 16-byte aligned; the row holds n rounded up to 4).
template <int PER>
__device__ __forceinline__ void load_chunk(const float *e, int c0, int n, float4 (&v)[PER / 4]) {
    static_assert(PER % 4 == 0, "float4 loads");
    const int last4 = ((n + 3) >> 2) - 1;
    const int b4 = (c0 + (int)threadIdx.x * PER) >> 2;
#pragma unroll
    for (int k = 0; k < PER / 4; k++) v[k] = reinterpret_cast<const float4 *>(e)[min(b4 + k, last4)];
}

// The running sum over terms e[i] (times scale when kSearch) for i in
// [c_begin, min(c_end, n)), from s, in chunks of kSmpThreads·PER terms: the
// scan steps of the file comment. kSearch: stops at the first i where r <
// the sum after term i, in `hit` (else -1). Every thread of the workgroup
// calls it; every value that steers it is uniform. ph: the step parity,
// which alternates over every step of the kernel (a step's minima are reset
// before its first barrier, the previous step's read after its second).
template <bool kSearch, int PER>
__device__ float grid_chain(const float *e, int c_begin, int c_end, int n, float scale, float s, float r, int &hit,
                            int &ph, const float4 (&first)[PER / 4], SmpLds &sm) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int kChunk = kSmpThreads * PER;
    const int end = min(c_end, n);
    hit = -1;
    // the first chunk's terms come loaded; each chunk's steps run while the
    // next chunk's loads are in flight
    float4 cur[PER / 4];
#pragma unroll
    for (int k = 0; k < PER / 4; k++) cur[k] = first[k];
    for (int c0 = c_begin; c0 < end; c0 += kChunk) {
        const int base = tid * PER;  // the thread's first position in the chunk
        const bool more = c0 + kChunk < end;
        float4 nxt[PER / 4];
        if (more) load_chunk<PER>(e, c0 + kChunk, n, nxt);
        float t[PER];
#pragma unroll
        for (int k = 0; k < PER / 4; k++) {
            t[4 * k] = cur[k].x;
            t[4 * k + 1] = cur[k].y;
            t[4 * k + 2] = cur[k].z;
            t[4 * k + 3] = cur[k].w;
        }
        if (kSearch) {
#pragma unroll
            for (int j = 0; j < PER; j++) t[j] = t[j] * scale;
        }
        const int valid_end = min(kChunk, end - c0);
        int from = 0;
        while (true) {
            // a NaN sum stays NaN, and r < NaN never holds
            if (s != s) return s;
            const Grid g = grid_of(s);
            // the thread's increments and events
            const int lo = from - base, hi = valid_end - base;
            uint32_t pre[PER], evm, acc;
            // one path a wave: every lane's positions valid, none, or a mix
            // (the checked path, right for any thread)
            const bool full = lo <= 0 && hi >= PER, none = lo >= PER || hi <= 0;
            const unsigned long long bfull = __ballot(full), bnone = __ballot(none);
            const unsigned long long all = __ballot(true);
            if (bfull == all) {
                acc = grid_terms<PER, false>(t, g, lo, hi, pre, evm);
            } else if (bnone != all) {
                acc = grid_terms<PER, true>(t, g, lo, hi, pre, evm);
            } else {
#pragma unroll
                for (int j = 0; j < PER; j++) pre[j] = 0;
                acc = 0;
                evm = 0;
            }
            // exclusive prefix of the threads' sums in the workgroup. A
            // thread's sum is taken at most 2^24 (a sum that large crosses
            // at or before the thread's end, so the positions after it need
            // no exact offset), and a wave's then stays below 2^31.
            const uint32_t tv = min(acc, kGridTop);
            const uint32_t incl = wave_scan_add(tv);
            const uint32_t ex = incl - tv;
            if (lane == 63) sm.wt[wave] = incl;
            if (tid == 0) {
                sm.emin[ph] = kNone;
                sm.hmin[ph] = kNone;
            }
            __syncthreads();
            uint32_t woff = 0, total = 0;
#pragma unroll
            for (int w = 0; w < kSmpWaves; w++) {
                const uint32_t x = sm.wt[w];
                woff = w < wave ? sat_add(woff, x) : woff;
                total = sat_add(total, x);
            }
            const uint32_t off = sat_add(woff, ex);
            // pre[] grows with j: the first position at or past a threshold
            // is the count of those below it. The sum after position j is
            // (m + off + pre[j])·2^eu; it leaves the grid at m + off +
            // pre[j] >= 2^24, and passes r at m + off + pre[j] > r·2^-eu.
            const uint32_t room = kGridTop - g.m;
            const uint32_t thr = off >= room ? 0u : room - off;
            uint32_t hthr = 0xFFFFFFFFu;
            if (kSearch) {
                // r >= s, so floor(r·2^-eu) >= m
                const float rq = __builtin_amdgcn_ldexpf(r, -g.eu);
                if (rq < 33554432.0f) {
                    const uint32_t need = (uint32_t)__builtin_floorf(rq) + 1u - g.m;
                    hthr = off >= need ? 0u : need - off;
                }
            }
            // (pre[PER-1] = acc: a thread whose end stays below a threshold
            // needs no count)
            int nc = thr == 0 ? 0 : PER, nh = hthr == 0 ? 0 : PER;
            if (thr != 0 && acc >= thr) {
                nc = 0;
#pragma unroll
                for (int j = 0; j < PER; j++) nc += pre[j] < thr ? 1 : 0;
            }
            if (kSearch && hthr != 0 && acc >= hthr) {
                nh = 0;
#pragma unroll
                for (int j = 0; j < PER; j++) nh += pre[j] < hthr ? 1 : 0;
            }
            const int jev = min(nc, evm ? (int)__builtin_ctz(evm) : PER);
            // the thread's first event, and the sum after it (exact when it
            // is the workgroup's first)
            int je = kNone, jh = kNone;
            float cand = 0.0f;
            if (jev < PER) {
                float tj = t[0];
                uint32_t pb = 0;
                if (jev > 0) {
#pragma unroll
                    for (int j = 1; j < PER; j++) {
                        tj = jev == j ? t[j] : tj;
                        pb = jev == j ? pre[j - 1] : pb;
                    }
                }
                je = base + jev;
                cand = grid_value(g.m + off + pb, g.eu) + tj;
            }
            if (kSearch && nh < jev) jh = base + nh;
            // Every position after a crossing or a hit qualifies too: only
            // the wave's first (its lowest such lane: positions grow with
            // the lane) takes part in the minimum.
            const unsigned long long be = __ballot(je != kNone);
            const unsigned long long bh = __ballot(jh != kNone);
            if (be && lane == (int)__builtin_ctzll(be)) atomicMin(&sm.emin[ph], je);
            if (bh && lane == (int)__builtin_ctzll(bh)) atomicMin(&sm.hmin[ph], jh);
            sm.cand[tid] = cand;
            __syncthreads();
            const int es = __builtin_amdgcn_readfirstlane(sm.emin[ph]);
            const int hs = __builtin_amdgcn_readfirstlane(sm.hmin[ph]);
            ph ^= 1;
            if (kSearch && hs < es) {
                hit = c0 + hs;
                return s;
            }
            if (es == kNone) {
                s = grid_value(g.m + total, g.eu);
                break;
            }
            s = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sm.cand[es / PER])));
            if (kSearch && r < s) {
                hit = c0 + es;
                return s;
            }
            from = es + 1;
            if (from >= valid_end) break;
        }
        if (more) {
#pragma unroll
            for (int k = 0; k < PER / 4; k++) cur[k] = nxt[k];
        }
    }
    return s;
}

// The running sum over all n terms (times scale when kSearch): the first
// kSmpPre one by one, then grid_chain. kSearch: the first i where r < the
// sum after term i, in `hit` (else -1).
template <bool kSearch>
__device__ float chain(const float *e, int n, float scale, float r, int &hit, int &ph, SmpLds &sm) {
    const int tid = threadIdx.x;
    const int np = min(n, kSmpPre);
    // the scan's first chunk, loading while the first terms are added
    float4 c4[1];
    if (n > kSmpPre) load_chunk<4>(e, kSmpPre, n, c4);
    // pads are +0: the sums past n repeat the last
    if (tid < kSmpPre) sm.pre[tid] = tid < np ? (kSearch ? e[tid] * scale : e[tid]) : 0.0f;
    if (tid == 0) sm.first = kNone;
    __syncthreads();
    if (tid == 0) lds_chain_cum(sm.pre, kSmpPre);
    __syncthreads();
    const float s = sm.pre[np - 1];
    hit = -1;
    if (kSearch) {
        // the sums grow with the position: the wave's lowest lane is its first
        const unsigned long long b = __ballot(tid < np && r < sm.pre[min(tid, kSmpPre - 1)]);
        if (b && (tid & 63) == (int)__builtin_ctzll(b)) atomicMin(&sm.first, tid);
        __syncthreads();
        const int f = sm.first;
        if (f != kNone) {
            hit = f;
            return s;
        }
    }
    __syncthreads();  // the prefix is read before grid_chain's LDS is reused
    // chunks of 1024, 4096, then 8192 terms: binade crossings are densest
    // early, and a step after an event rescans the rest of its chunk
    static_assert(kSmpThreads == 256, "the chunk schedule");
    float x = grid_chain<kSearch, 4>(e, kSmpPre, kSmpPre + 1024, n, scale, s, r, hit, ph, c4, sm);
    if (hit >= 0 || n <= kSmpPre + 1024) return x;
    float4 c16[4];
    load_chunk<16>(e, kSmpPre + 1024, n, c16);
    x = grid_chain<kSearch, 16>(e, kSmpPre + 1024, kSmpPre + 5120, n, scale, x, r, hit, ph, c16, sm);
    if (hit >= 0 || n <= kSmpPre + 5120) return x;
    float4 c32[8];
    load_chunk<32>(e, kSmpPre + 5120, n, c32);
    return grid_chain<kSearch, 32>(e, kSmpPre + 5120, n, n, scale, x, r, hit, ph, c32, sm);
}

// The greedy argmax of a row (sample.go:45-53): the first index holding the
// largest value; NaNs are never candidates, and a NaN first logit (or every
// logit NaN) gives index 0, as the reference's `>` scan does. Valid in
// thread 0; every thread calls it.
template <int NT>
__device__ int wg_argmax(const float *row, int64_t vocab, float *s_v, int *s_i) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float bv = 0.0f;
    int bi = -1;
    // eight 16-byte loads in flight a thread (a position past the row
    // re-reads the last group: merging an element twice changes nothing)
    const int64_t n4 = (reinterpret_cast<uintptr_t>(row) & 15) == 0 ? vocab >> 2 : 0;
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    for (int64_t b = threadIdx.x; b < n4; b += NT * 8) {
        float4 v[8];
        int64_t g[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            g[u] = min(b + NT * u, n4 - 1);
            v[u] = r4[g[u]];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
            for (int c = 0; c < 4; c++)
                if (e[c] == e[c]) argmax_merge(bv, bi, e[c], (int)(4 * g[u] + c));
        }
    }
    for (int64_t i = 4 * n4 + threadIdx.x; i < vocab; i += NT) {
        const float v = row[i];
        if (v == v) argmax_merge(bv, bi, v, (int)i);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_down(bv, off);
        const int oi = __shfl_down(bi, off);
        argmax_merge(bv, bi, ov, oi);
    }
    if (lane == 0) {
        s_v[wave] = bv;
        s_i[wave] = bi;
    }
    __syncthreads();
    float v = 0.0f;
    int i = -1;
    if (threadIdx.x == 0) {
        for (int w = 0; w < NT / 64; w++) argmax_merge(v, i, s_v[w], s_i[w]);
        if (row[0] != row[0] || i < 0) i = 0;
    }
    return i;
}

// Whether sequence z picks a token this step: its logits are those of
// position pos[z], and the token at pos[z]+1 is past its prompt and inside
// the tokens row.
__device__ __forceinline__ bool picks(const int32_t *pos, const int32_t *prompt, int z, int32_t tokens_len) {
    const int p = pos[z];
    return p + 1 >= prompt[z] && p + 1 < tokens_len;
}

// Go max of logit_i / T over a slice of the row, one partial a workgroup.
__global__ __launch_bounds__(kSmpPartThreads) void sample_max_kernel(const float *logits, int64_t vocab,
                                                                     const int32_t *pos, const int32_t *prompt,
                                                                     int32_t tokens_len, const float *temps,
                                                                     float *part) {
    __shared__ float s_m[kSmpPartThreads / 64];
    const int z = blockIdx.y;
    const float T = temps[z];
    if (!picks(pos, prompt, z, tokens_len) || T <= 0) return;
    const float *row = logits + (int64_t)z * vocab;
    constexpr int64_t kStride = (int64_t)kSmpParts * kSmpPartThreads;
    float m = row[0] / T;
    // four loads in flight a thread (a position past the row re-reads row[0])
    for (int64_t i0 = (int64_t)blockIdx.x * kSmpPartThreads + threadIdx.x; i0 < vocab; i0 += 4 * kStride) {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = row[i0 + k * kStride < vocab ? i0 + k * kStride : 0];
#pragma unroll
        for (int k = 0; k < 4; k++) m = gomax(m, v[k] / T);
    }
    m = wave_gomax(m);
    if ((threadIdx.x & 63) == 0) s_m[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float x = s_m[0];
        for (int w = 1; w < kSmpPartThreads / 64; w++) x = gomax(x, s_m[w]);
        part[z * kSmpParts + blockIdx.x] = x;
    }
}

// e_i = Exp32(logit_i / T - mx) over a slice of the row, mx the Go max of
// the partials.
__global__ __launch_bounds__(kSmpPartThreads) void sample_terms_kernel(const float *logits, int64_t vocab,
                                                                       int64_t estride, const int32_t *pos,
                                                                       const int32_t *prompt, int32_t tokens_len,
                                                                       const float *temps, const float *part,
                                                                       float *terms) {
    const int z = blockIdx.y;
    const float T = temps[z];
    if (!picks(pos, prompt, z, tokens_len) || T <= 0) return;
    static_assert(kSmpParts % 64 == 0, "partials a lane");
    const float *pz = part + (int64_t)z * kSmpParts + (threadIdx.x & 63);
    float mx = pz[0];
#pragma unroll
    for (int k = 1; k < kSmpParts / 64; k++) mx = gomax(mx, pz[64 * k]);
    mx = wave_gomax(mx);
    const float *row = logits + (int64_t)z * vocab;
    float *e = terms + (int64_t)z * estride;
    constexpr int64_t kStride = (int64_t)kSmpParts * kSmpPartThreads;
    for (int64_t i0 = (int64_t)blockIdx.x * kSmpPartThreads + threadIdx.x; i0 < vocab; i0 += 4 * kStride) {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = row[i0 + k * kStride < vocab ? i0 + k * kStride : 0];
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (i0 + k * kStride < vocab) e[i0 + k * kStride] = exp32(v[k] / T - mx);
    }
}

// One workgroup a sequence: the token at pos[z]+1 (the argmax when T <= 0,
// else the draw), written when the sequence picks one, and pos[z] advances.
// amax (one sequence): the classifier's argmax keys, cleared for the next
// product.
__global__ __launch_bounds__(kSmpThreads) void sample_pick_kernel(const float *logits, const float *terms,
                                                                  int64_t vocab, int64_t estride, int32_t *pos,
                                                                  const int32_t *prompt, int32_t *tokens,
                                                                  int64_t tok_stride, int32_t tokens_len,
                                                                  const float *temps, uint64_t *states,
                                                                  unsigned long long *amax) {
    __shared__ SmpLds sm;
    const int z = blockIdx.x, tid = threadIdx.x;
    if (amax && tid < kArgmaxSlots) amax[tid] = 0ull;
    const int p = pos[z];
    const bool pick = picks(pos, prompt, z, tokens_len);
    const float T = temps[z];
    int token = 0;
    if (pick && T <= 0) {
        token = wg_argmax<kSmpThreads>(logits + (int64_t)z * vocab, vocab, sm.bv, sm.bi);
    } else if (pick) {
        const int n = (int)vocab;
        const float *e = terms + (int64_t)z * estride;
        int hit, ph = 0;
        const float S = chain<false>(e, n, 1.0f, 0.0f, hit, ph, sm);
        const float inv = recip32(S);
        // the draw (sample.go:18-24), after the softmax as the reference
        // takes it; the state advances once a sampled token
        if (tid == 0) {
            uint64_t st = states[z];
            st ^= st >> 12;
            st ^= st << 25;
            st ^= st >> 27;
            states[z] = st;
            sm.r = (float)((st * 0x2545f4914f6cdd1dull) >> 40) / (float)(1 << 24);
        }
        __syncthreads();
        const float r = sm.r;
        chain<true>(e, n, inv, r, hit, ph, sm);
        token = hit >= 0 ? hit : n - 1;
    }
    __syncthreads();  // every thread has read pos[z] before it moves
    if (tid == 0) {
        if (pick) tokens[(int64_t)z * tok_stride + p + 1] = token;
        pos[z] = p + 1;
    }
}

// Independent sequences' greedy step (sample.go:45-53 per sequence):
// workgroup z writes the argmax of logits row z as the token at pos[z]+1
// when that position is past the prompt, and advances pos[z].
__global__ __launch_bounds__(1024) void seqs_advance_kernel(const float *logits, int64_t vocab, int32_t *pos,
                                                            const int32_t *prompt, int32_t *tokens,
                                                            int64_t tok_stride, int32_t tokens_len) {
    __shared__ float s_v[16];
    __shared__ int s_i[16];
    const int z = blockIdx.x;
    const int i = wg_argmax<1024>(logits + (int64_t)z * vocab, vocab, s_v, s_i);
    if (threadIdx.x == 0) {
        const int p = pos[z];
        if (p + 1 >= prompt[z] && p + 1 < tokens_len) tokens[(int64_t)z * tok_stride + p + 1] = i;
        pos[z] = p + 1;
    }
}

}  // namespace

void launch_seqs_advance(const float *logits, int64_t vocab, int seqs, int32_t *pos, const int32_t *prompt,
                         int32_t *tokens, int64_t tok_stride, int32_t tokens_len, hipStream_t s) {
    RK_LAUNCH(seqs_advance_kernel, dim3(seqs), dim3(1024), 0, s, logits, vocab, pos, prompt, tokens, tok_stride,
              tokens_len);
}

int64_t sample_terms_stride(int64_t vocab) { return (vocab + 3) & ~(int64_t)3; }

int sample_parts() { return kSmpParts; }

void launch_sample(const SampleArgs &a, hipStream_t s) {
    RK_LAUNCH(sample_max_kernel, dim3(kSmpParts, a.seqs), dim3(kSmpPartThreads), 0, s, a.logits, a.vocab, a.pos,
              a.prompt, a.tokens_len, a.temps, a.part);
    const int64_t es = sample_terms_stride(a.vocab);
    RK_LAUNCH(sample_terms_kernel, dim3(kSmpParts, a.seqs), dim3(kSmpPartThreads), 0, s, a.logits, a.vocab, es, a.pos,
              a.prompt, a.tokens_len, a.temps, a.part, a.terms);
    RK_LAUNCH(sample_pick_kernel, dim3(a.seqs), dim3(kSmpThreads), 0, s, a.logits, a.terms, a.vocab, es, a.pos,
              a.prompt, a.tokens, a.tok_stride, a.tokens_len, a.temps, a.states, a.amax);
}

}  // namespace rk

using namespace rk;

// Sampler.Sample over rows of host logits (internal/llm/sample.go:26-43):
// row z with temperature[z] and the generator state state[z] (updated).
extern "C" int rk_sample_logits(rk_device *d, const float *logits, int64_t vocab, int32_t rows,
                                const float *temperature, uint64_t *state, int32_t *tokens) {
    if (!d || vocab <= 0 || vocab > INT32_MAX || rows < 0 || (rows > 0 && (!logits || !temperature || !state || !tokens)))
        return fail(d, RK_ERR_ARGS, "rk_sample_logits: bad arguments");
    if (rows == 0) return RK_OK;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    // logits, terms, partials and temperatures (floats), then the states,
    // and the positions, prompt lengths and tokens (int32)
    const int64_t nl = vocab * rows, nl_pad = (nl + 63) & ~(int64_t)63;
    const int64_t nt = sample_terms_stride(vocab) * rows, np = (int64_t)sample_parts() * rows;
    const int64_t nf = nl_pad + nt + np + ((rows + 63) & ~63);
    const size_t bytes = (size_t)4 * nf + (size_t)8 * rows + (size_t)4 * 4 * rows;
    char *buf = nullptr;
    int rc = dev_alloc(d, (void **)&buf, bytes, "sample");
    if (rc) return rc;
    float *f = reinterpret_cast<float *>(buf);
    uint64_t *st = reinterpret_cast<uint64_t *>(buf + (size_t)4 * nf);
    int32_t *pos = reinterpret_cast<int32_t *>(st + rows), *prompt = pos + rows, *tok = prompt + rows;
    SampleArgs a{};
    a.logits = f;
    a.terms = f + nl_pad;
    a.part = a.terms + nt;
    a.temps = a.part + np;
    a.vocab = vocab;
    a.seqs = rows;
    a.states = st;
    // every row picks the token at position 1 of its two-entry row
    a.pos = pos;
    a.prompt = prompt;
    a.tokens = tok;
    a.tok_stride = 2;
    a.tokens_len = 2;
    hipStream_t s = d->stream;
    hipError_t e = hipMemsetAsync(pos, 0, (size_t)4 * 4 * rows, s);
    if (e == hipSuccess) e = hipMemcpyAsync(f, logits, (size_t)4 * nl, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync((void *)a.temps, temperature, (size_t)4 * rows, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(st, state, (size_t)8 * rows, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) {
        launch_sample(a, s);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpyAsync(state, st, (size_t)8 * rows, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(tokens, 4, tok + 1, 8, 4, (size_t)rows, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(buf);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return hip_fail(d, e, "rk_sample_logits");
    }
    return RK_OK;
}
