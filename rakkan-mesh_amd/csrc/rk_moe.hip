// rk_moe.hip — a mixture-of-experts feed-forward on the device (config 5,
// Qwen3-MoE shape). The reference has no llama-family MoE; the contract is
// this build's, after the dsv41 precedent (internal/llm/dsv41/ops.go:67-74
// topK, forward.go:355-413 moe), for each token's RMS-normed input xn:
//
//   z = router·xn                       Q8 product, MatVecQ8's bits
//   p = softmax(z)                      Go max, Exp32, one sequential sum,
//                                       Recip32 (internal/llm/model.go:640-654)
//   sel = topK(p, k)                    stable by cmp.Compare: larger first,
//                                       lower index on ties, NaN last
//   w_i = p_sel_i·Recip32(Σ_i p_sel_i)  the sum in selection order
//   h = float32(w·float32(silu(W1·xn)·(W3·xn)))  per selected expert
//   y = Σ W2·h over the selected experts in ascending index, from +0
//
// Launches: the router's product (on the quantized input; a batch of up to
// 16 tokens a row per wave, the tokens' codes in LDS); the routing (one wave
// per token) and the grouping of the (token, slot) pairs by expert (counts
// and places in parallel for up to 128 pairs), one launch for up to 16
// tokens; each selected expert's W1/W3 rows for all the tokens that chose
// it, with the gate, the weight and h's quantization; each selected
// expert's W2 rows for those tokens; the ascending-order sum (optionally
// into a residual). One token with its RMSNorm (a decode step): the router
// with the norm in its prologue, the W1/W3 kernel routing the token itself,
// and W2 with the sum: three launches.
// An expert's rows are read from memory once per call however many tokens
// chose it: a wave loads a chunk of its rows and dots it with each of the
// group's inputs. Every expert product is a row dot of MatVecQ8 (integer
// block sums, the eight ordered running sums), so each token's bits do not
// depend on the batch or on the grouping.
#include <algorithm>
#include <mutex>
#include <vector>

#include "rk_dev.h"
#include "rk_fused.h"
#include "rk_mm.h"
#include "rk_moe.h"
#include "rk_sync.h"

namespace rk {

namespace {

constexpr int kMoeMaxK = 32;        // experts per token
constexpr int kMoeMaxExperts = 1024;
constexpr int kMoeMaxCols = 8192;   // widest expert input (chunks of 1 KiB per row)
constexpr int kMoePass = 4;         // inputs an expert's rows meet per pass

// NR Q8 rows dotted with np (<= NP) quantized inputs, each (row, input) in
// MatVecQ8's order: exact block sums; block b into running sum b mod 8 in
// order of b; the fixed tree ((0+1)+(2+3))+((4+5)+(6+7)). Each chunk of the
// rows is loaded once for all the inputs. Lane 0 returns res[j][r]. Every
// lane of the wave calls it; np is wave-uniform.
template <int NR, int NP>
__device__ __forceinline__ void wave_rows_q8_multi(const uint8_t *const (&w)[NR], const float *const (&ws)[NR],
                                                   const int8_t *const (&qx)[NP], const float *const (&xs)[NP], int np,
                                                   int cols, float (&res)[NP][NR]) {
    const int lane = threadIdx.x & 63;
    const int nb = cols >> 5, C = (cols + 1023) >> 10;
    float acc[NP][NR];
#pragma unroll
    for (int j = 0; j < NP; j++)
#pragma unroll
        for (int r = 0; r < NR; r++) acc[j][r] = 0.0f;
    for (int c = 0; c < C; c++) {
        const int o = min(c * 1024 + lane * 16, cols - 16);  // lanes past the row's end: blocks excluded below
        int4 wv[NR];
        float sw[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            wv[r] = load_stream16_g(w[r] + o);  // (table pointers: global loads, not flat)
            sw[r] = loadf_g(ws[r] + (o >> 5));
        }
        const int b0 = c * 32 + (lane >> 1);
#pragma unroll
        for (int j = 0; j < NP; j++) {
            if (j >= np) break;  // uniform
            const int4 xv = *reinterpret_cast<const int4 *>(qx[j] + o);
            const float sx = xs[j][o >> 5];
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const int s = pair_sum(dot16(wv[r], xv, 0));
                const float t = (float)s * (sw[r] * sx);
                // block 32c+k is in lanes 2k, 2k+1; running sum L (lane 2L)
                // takes blocks 32c+L, +8, +16, +24
                const float t1 = __shfl_down(t, 16), t2 = __shfl_down(t, 32), t3 = __shfl_down(t, 48);
                if (lane < 16 && (lane & 1) == 0) {
                    if (b0 < nb) acc[j][r] += t;
                    if (b0 + 8 < nb) acc[j][r] += t1;
                    if (b0 + 16 < nb) acc[j][r] += t2;
                    if (b0 + 24 < nb) acc[j][r] += t3;
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < NP; j++)
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const float p2 = acc[j][r] + __shfl_down(acc[j][r], 2);
            const float q4 = p2 + __shfl_down(p2, 4);
            res[j][r] = q4 + __shfl_down(q4, 8);
        }
}

// The router's product for a batch of up to kRouterMaxT tokens (their codes
// and scales in LDS): wave w of workgroup b takes row 4b + w (MatVecQ8's bits)
// for every token, eight tokens a pass; lane l keeps, for token l/8 of the
// pass, running sum l mod 8 (blocks l mod 8, +8, ... in order), so the sums
// need no lane exchanges until the fixed tree ((0+1)+(2+3))+((4+5)+(6+7)).
// The row's blocks are loaded once, up front; the tokens' codes are staged
// in LDS. logits: [tokens][experts].
constexpr int kRouterBpl = 8;  // blocks of a row per lane (rows up to 2048 wide)
constexpr int kRouterMaxT = 16;
__global__ __launch_bounds__(256) void moe_router_rows_kernel(const uint8_t *rw, const float *rws, int experts, int dim,
                                                              const int8_t *qx, const float *xs, int tokens,
                                                              float *logits) {
    extern __shared__ __align__(16) char rlds[];
    int8_t *sq = reinterpret_cast<int8_t *>(rlds);                             // [tokens][dim] codes
    float *sxs = reinterpret_cast<float *>(rlds + (int64_t)tokens * dim);   // [tokens][dim/32] scales
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rl = lane & 7, tg = lane >> 3;
    const int nb = dim >> 5;
    const int rowi = blockIdx.x * 4 + wave, row = min(rowi, experts - 1);
    const uint8_t *rp = rw + (int64_t)row * dim;
    const float *rs = rws + (int64_t)row * nb;
    int4 c0[kRouterBpl], c1[kRouterBpl];
    float sw[kRouterBpl];
    lane_row_load<kRouterBpl>(c0, c1, sw, rp, rs, nb, rl);
    for (int i = tid; i < (tokens * dim) >> 4; i += 256)
        reinterpret_cast<int4 *>(sq)[i] = reinterpret_cast<const int4 *>(qx)[i];
    for (int i = tid; i < tokens * nb; i += 256) sxs[i] = xs[i];
    __syncthreads();
    if (rowi >= experts) return;  // uniform over the wave
    for (int t0 = 0; t0 < tokens; t0 += 8) {
        const int t = min(t0 + tg, tokens - 1);
        const float acc = tree8(lane_running_sum<kRouterBpl>(c0, c1, sw, sq + t * dim, sxs + t * nb, nb, rl));
        if (rl == 0 && t0 + tg < tokens) logits[(int64_t)(t0 + tg) * experts + row] = acc;
    }
}

// 64-bit key of probability v at expert e for a max-reduction that picks
// what a stable sort by cmp.Compare puts first: order-preserving value bits
// above (-0 as +0; NaN lowest of all), the complement of the index below.
// Never 0, so 0 marks a taken entry.
__device__ __forceinline__ unsigned long long route_key(float v, int e) {
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    if (v != v) u = 0;
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)e);
}

__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long k, int ctrl_tag) {
    uint32_t lo = (uint32_t)k, hi = (uint32_t)(k >> 32);
    switch (ctrl_tag) {  // the DPP control must be a constant
        case 0: lo = __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xF, 0xF, false); hi = __builtin_amdgcn_mov_dpp(hi, 0xB1, 0xF, 0xF, false); break;
        case 1: lo = __builtin_amdgcn_mov_dpp(lo, 0x4E, 0xF, 0xF, false); hi = __builtin_amdgcn_mov_dpp(hi, 0x4E, 0xF, 0xF, false); break;
        case 2: lo = __builtin_amdgcn_mov_dpp(lo, 0x141, 0xF, 0xF, false); hi = __builtin_amdgcn_mov_dpp(hi, 0x141, 0xF, 0xF, false); break;
        default: lo = __builtin_amdgcn_mov_dpp(lo, 0x140, 0xF, 0xF, false); hi = __builtin_amdgcn_mov_dpp(hi, 0x140, 0xF, 0xF, false); break;
    }
    return ((unsigned long long)hi << 32) | lo;
}

// Largest key over the wave, valid in every lane: rows of 16 by DPP, then
// the four rows by readlane. Every lane of the wave must call it.
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const unsigned long long o = dpp_u64(k, c);
        k = o > k ? o : k;
    }
    unsigned long long best = 0;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)k, 16 * r);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(k >> 32), 16 * r);
        const unsigned long long v = ((unsigned long long)hi << 32) | lo;
        best = v > best ? v : best;
    }
    return best;
}

constexpr int kRoutePer = kMoeMaxExperts / 64;  // experts per lane at most

// Routing of one token by one wave: softmax, stable top-k, normalized
// weights, written to sel/wsel [k] (when not null). Every thread of the
// workgroup calls it (its barrier is the workgroup's); `live` false: a wave
// without a token, which only takes part in the barrier. z: the token's
// logits (global or LDS); sp: [experts] floats of LDS, 16-byte aligned (may
// be z itself). Lane r < k of a live wave returns the r-th selected expert
// and its weight (wt). PER: experts a lane holds (experts <= 64·PER).
template <int PER>
__device__ int route_wave(bool live, const float *z, int experts, int k, float *sp, int32_t *sel, float *wsel,
                          float &wt) {
    const int lane = threadIdx.x & 63;
    float m = live ? z[0] : 0.0f;
    if (live)
        for (int e = lane; e < experts; e += 64) {
            const float v = z[e];
            sp[e] = v;
            m = gomax(m, v);
        }
    m = wave_gomax(m);
    if (live)
        for (int e = lane; e < experts; e += 64) sp[e] = exp32(sp[e] - m);
    __syncthreads();
    // the one sequential sum: every lane runs the same chain (the reads
    // broadcast), so the result is the same in all lanes
    const float inv = live ? recip32(lds_chain_sum(sp, experts, 0.0f)) : 0.0f;
    unsigned long long key[PER];
    float pv[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = lane + 64 * j;
        key[j] = 0;
        pv[j] = 0.0f;
        if (live && e < experts) {
            pv[j] = sp[e] * inv;
            key[j] = route_key(pv[j], e);
        }
    }
    // top-k: k rounds of the largest remaining key; lane r keeps round r's
    int mine = 0;
    for (int r = 0; r < k; r++) {
        unsigned long long b = 0;
#pragma unroll
        for (int j = 0; j < PER; j++) b = key[j] > b ? key[j] : b;
        b = wave_max_u64(b);
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (key[j] == b) key[j] = 0;
        if (lane == r) mine = (int)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull));
    }
    // each selected expert's probability, from the lane that holds it
    float ps = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        if (64 * j < experts) {  // uniform
            const float v = __shfl(pv[j], mine & 63);
            if ((mine >> 6) == j) ps = v;
        }
    }
    // their sum in selection order, from +0 (the same in every lane)
    float sum = 0.0f;
    for (int r = 0; r < k; r++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ps), r));
    const float inv2 = recip32(sum);
    wt = ps * inv2;
    if (live && lane < k && sel) {
        sel[lane] = mine;
        wsel[lane] = wt;
    }
    return mine;
}

// Routing of one token per workgroup (one wave).
template <int PER>
__global__ __launch_bounds__(64) void moe_route_kernel(const float *logits, int experts, int k, int32_t *sel,
                                                       float *wsel) {
    extern __shared__ __align__(16) float sp[];  // [experts] probabilities
    const int t = blockIdx.x;
    float wt;
    (void)route_wave<PER>(true, logits + (int64_t)t * experts, experts, k, sp, sel + (int64_t)t * k,
                          wsel + (int64_t)t * k, wt);
}

// The experts' row tables, and group g's rows written beside the grouping
// (so the expert kernels find their rows with one load, not two).
struct MoeTabs {
    const uint8_t *const *w1, *const *w3, *const *w2;
    const float *const *s1, *const *s3, *const *s2;
    // optional counters: the experts selected (summed over groupings), and
    // the groupings (MoeScratch::stat)
    unsigned long long *stat;
};
// Thread e's expert's six row addresses, read at a kernel's start (they
// do not depend on the routing) so they are in registers by the time the
// grouping writes them.
struct ExpRows {
    const void *p[6];
};
__device__ __forceinline__ ExpRows expert_rows(const MoeTabs &tb, int e, int experts) {
    ExpRows r{};
    if (e < experts) {
        r.p[0] = tb.w1[e];
        r.p[1] = tb.s1[e];
        r.p[2] = tb.w3[e];
        r.p[3] = tb.s3[e];
        r.p[4] = tb.w2[e];
        r.p[5] = tb.s2[e];
    }
    return r;
}
__device__ __forceinline__ void group_rows(const ExpRows &r, int g, const void **gptr) {
    const void **d = gptr + 6 * g;
#pragma unroll
    for (int i = 0; i < 6; i++) d[i] = r.p[i];
}

constexpr int kGroupFastPairs = 128;
struct GroupLds {
    int cnt[1024], start[1024], gi[1024], total;
};

// The scans over the experts' counts (one wave; lane l takes experts
// l·per .. l·per+per-1: local sums, then an exclusive scan of the lane
// totals across the wave): each expert's first place and group index, and
// the number of groups. Then each selected expert's group entry and rows.
// Every thread of a 1024-thread workgroup calls it, after the counts.
__device__ void group_scan_info(GroupLds &gl, int experts, int gcap, int32_t *grp, const ExpRows &rows,
                                const void **gptr, unsigned long long *stat) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) {
        const int per = (experts + 63) / 64;
        int c = 0, g = 0;
        for (int i = 0; i < per; i++) {
            const int e = lane * per + i;
            if (e < experts) {
                c += gl.cnt[e];
                g += gl.cnt[e] > 0;
            }
        }
        int ci = c, gi = g;  // inclusive scans
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int oc = __shfl_up(ci, d), og = __shfl_up(gi, d);
            if (lane >= d) {
                ci += oc;
                gi += og;
            }
        }
        int cs = ci - c, gs = gi - g;  // exclusive
        for (int i = 0; i < per; i++) {
            const int e = lane * per + i;
            if (e < experts) {
                gl.start[e] = cs;
                gl.gi[e] = gs;
                cs += gl.cnt[e];
                gs += gl.cnt[e] > 0;
            }
        }
        if (lane == 63) gl.total = gi;
    }
    __syncthreads();
    int32_t *gexp = grp + 1, *gstart = grp + 1 + gcap, *gcount = grp + 1 + 2 * gcap;
    if (tid < experts && gl.cnt[tid] > 0) {
        const int g = gl.gi[tid];
        gexp[g] = tid;
        gstart[g] = gl.start[tid];
        gcount[g] = gl.cnt[tid];
        group_rows(rows, g, gptr);
    }
    if (tid == 0) {
        grp[0] = gl.total;
        if (stat) {
            atomicAdd(&stat[0], (unsigned long long)gl.total);
            atomicAdd(&stat[1], 1ull);
        }
    }
}

// The (token, slot) pairs grouped by expert: grp[0] = the number of experts
// selected, then at grp + 1 + g, + gcap, + 2·gcap their index (ascending),
// first entry in the pair list and count, and the pair list from
// grp + 1 + 3·gcap, with the listed pairs' weights in gwt and each group's
// rows in gptr. One workgroup, any number of pairs: counts by LDS atomics,
// the scans, then each pair's place by a ticket of its expert's count. The
// order of a group's pairs is then not fixed; no result depends on it (each
// pair's products are its own, and the sum over a token's experts follows
// the experts' order).
__global__ __launch_bounds__(1024) void moe_group_kernel(const int32_t *sel, const float *wsel, int npairs,
                                                         int experts, int gcap, int32_t *grp, float *gwt, MoeTabs tb,
                                                         const void **gptr) {
    __shared__ GroupLds gl;
    __shared__ int fill[1024];
    const int tid = threadIdx.x;
    const ExpRows rows = expert_rows(tb, tid, experts);
    gl.cnt[tid] = 0;
    fill[tid] = 0;
    __syncthreads();
    for (int p = tid; p < npairs; p += 1024) atomicAdd(&gl.cnt[sel[p]], 1);
    __syncthreads();
    group_scan_info(gl, experts, gcap, grp, rows, gptr, tb.stat);
    int32_t *list = grp + 1 + 3 * gcap;
    for (int p = tid; p < npairs; p += 1024) {
        const int e = sel[p];
        const float w = wsel[p];
        const int at = gl.start[e] + atomicAdd(&fill[e], 1);
        list[at] = p;
        gwt[at] = w;
    }
}

// The same grouping for up to kGroupFastPairs pairs and 1024 experts, with
// no thread walking all the pairs: counts by LDS atomics, one wave's scans
// over the experts (starts and group indices), and each pair's place among
// its expert's pairs from the earlier pairs (eight threads a pair). Every
// thread of a 1024-thread workgroup calls it; s_sel: the pairs' experts in
// LDS, written before a barrier.
__device__ void group_pairs_wg(const int *s_sel, const float *s_wt, int npairs, int experts, int gcap, int32_t *grp,
                               float *gwt, const ExpRows &rows, const void **gptr, GroupLds &gl,
                               unsigned long long *stat) {
    const int tid = threadIdx.x;
    gl.cnt[tid] = 0;
    __syncthreads();
    if (tid < npairs) atomicAdd(&gl.cnt[s_sel[tid]], 1);
    __syncthreads();
    group_scan_info(gl, experts, gcap, grp, rows, gptr, stat);
    // pair p's place: the earlier pairs of its expert (eight threads a pair)
    int32_t *list = grp + 1 + 3 * gcap;
    const int p = tid >> 3, part = tid & 7;
    if (p < npairs) {  // whole groups of eight
        const int e = s_sel[p];
        int n = 0;
        for (int q = part; q < p; q += 8) n += s_sel[q] == e;
        n += dpp_x1(n);
        n += dpp_x2(n);
        n += dpp_mirror8(n);
        if (part == 0) {
            list[gl.start[e] + n] = p;
            gwt[gl.start[e] + n] = s_wt[p];
        }
    }
}

__global__ __launch_bounds__(1024) void moe_group_fast_kernel(const int32_t *sel, const float *wsel, int npairs,
                                                              int experts, int gcap, int32_t *grp, float *gwt,
                                                              MoeTabs tb, const void **gptr) {
    __shared__ int s_sel[kGroupFastPairs];
    __shared__ float s_wt[kGroupFastPairs];
    __shared__ GroupLds gl;
    const ExpRows rows = expert_rows(tb, threadIdx.x, experts);
    if ((int)threadIdx.x < npairs) {
        s_sel[threadIdx.x] = sel[threadIdx.x];
        s_wt[threadIdx.x] = wsel[threadIdx.x];
    }
    __syncthreads();
    group_pairs_wg(s_sel, s_wt, npairs, experts, gcap, grp, gwt, rows, gptr, gl, tb.stat);
}

// Routing (wave t: token t) and grouping of up to kSelectTokens tokens in
// one workgroup. sp: [tokens][ep] probabilities (ep: experts rounded up to 4).
constexpr int kSelectTokens = 16;
template <int PER>
__global__ __launch_bounds__(1024) void moe_select_kernel(const float *logits, int tokens, int experts, int k,
                                                          int32_t *sel, float *wsel, int gcap, int32_t *grp,
                                                          float *gwt, MoeTabs tb, const void **gptr) {
    extern __shared__ __align__(16) float sp_all[];
    __shared__ int s_sel[kGroupFastPairs];
    __shared__ float s_wt[kGroupFastPairs];
    __shared__ GroupLds gl;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const ExpRows rows = expert_rows(tb, threadIdx.x, experts);
    const int ep = (experts + 3) & ~3;
    const bool live = wave < tokens;
    const int t = live ? wave : 0;
    float wt;
    const int mine = route_wave<PER>(live, logits + (int64_t)t * experts, experts, k, sp_all + t * ep,
                                     sel + (int64_t)t * k, wsel + (int64_t)t * k, wt);
    if (live && lane < k) {
        s_sel[t * k + lane] = mine;
        s_wt[t * k + lane] = wt;
    }
    __syncthreads();
    group_pairs_wg(s_sel, s_wt, tokens * k, experts, gcap, grp, gwt, rows, gptr, gl, tb.stat);
}

// W1 and W3 rows of a selected expert for every pair that chose it:
// h = w·(silu(W1·xn)·(W3·xn)), then h's Q8_0 block. Workgroup (group, block
// of 32 hidden rows), eight waves of four hidden rows (W1 and W3 of each:
// eight row dots), the group's pairs kMoePass at a time. Groups past the
// count exit.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void moe_up_kernel(const uint8_t *const *w1, const float *const *s1,
                                                     const uint8_t *const *w3, const float *const *s3,
                                                     const int32_t *grp, int gcap, const float *wsel, int k,
                                                     const int8_t *qx, const float *xs, int dim, int hidden,
                                                     int8_t *hq, float *hs, int32_t *hsum) {
    __shared__ __align__(16) float sh[kMoePass][32];
    const int g = blockIdx.x;
    if (g >= grp[0]) return;  // uniform
    const int e = grp[1 + g], start = grp[1 + gcap + g], count = grp[1 + 2 * gcap + g];
    const int32_t *list = grp + 1 + 3 * gcap + start;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j0 = blockIdx.y * 32 + 4 * wave;  // hidden rows j0 .. j0+3
    const int nb = dim >> 5;
    const uint8_t *w[8];
    const float *ws[8];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int j = j0 + q;  // hidden is a multiple of 32
        w[2 * q] = w1[e] + (int64_t)j * dim;
        ws[2 * q] = s1[e] + (int64_t)j * nb;
        w[2 * q + 1] = w3[e] + (int64_t)j * dim;
        ws[2 * q + 1] = s3[e] + (int64_t)j * nb;
    }
    for (int p0 = 0; p0 < count; p0 += kMoePass) {
        const int np = min(kMoePass, count - p0);
        int pr[kMoePass];
        const int8_t *xq[kMoePass];
        const float *xsp[kMoePass];
#pragma unroll
        for (int j = 0; j < kMoePass; j++) {
            pr[j] = list[p0 + min(j, np - 1)];
            const int t = pr[j] / k;
            xq[j] = qx + (int64_t)t * dim;
            xsp[j] = xs + (int64_t)t * nb;
        }
        float res[kMoePass][8];
        wave_rows_q8_multi<8, kMoePass>(w, ws, xq, xsp, np, dim, res);
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < kMoePass; j++) {
                if (j >= np) break;
                const float wt = wsel[pr[j]];
#pragma unroll
                for (int q = 0; q < 4; q++) sh[j][4 * wave + q] = wt * silu_mul(res[j][2 * q], res[j][2 * q + 1]);
            }
        }
        __syncthreads();
        if (wave < np) {  // pair `wave`'s block of h: lanes 0-7, four values each
            const int gi = min(lane, 7);
            const float4 v4 = reinterpret_cast<const float4 *>(sh[wave])[gi];
            float d;
            int cs;
            const uint32_t pk = quantize_group(v4.x, v4.y, v4.z, v4.w, d, cs);
            int p = pr[0];
#pragma unroll
            for (int j = 1; j < kMoePass; j++)
                if (j == wave) p = pr[j];
            const int64_t base = (int64_t)p * hidden + blockIdx.y * 32;
            if (lane < 8) {
                reinterpret_cast<uint32_t *>(hq + base)[lane] = pk;
                if (lane == 0) {
                    hs[base >> 5] = d;
                    hsum[base >> 5] = cs;
                }
            }
        }
        __syncthreads();
    }
}

// W2 rows of a selected expert on the quantized h of every pair that chose
// it. Workgroup (group, block of 16 output rows), four rows a wave.
constexpr int kDownRows = 4;
__global__ __launch_bounds__(256) void moe_down_kernel(const uint8_t *const *w2, const float *const *s2,
                                                       const int32_t *grp, int gcap, const int8_t *hq, const float *hs,
                                                       int dim, int hidden, float *o) {
    const int g = blockIdx.x;
    if (g >= grp[0]) return;  // uniform
    const int e = grp[1 + g], start = grp[1 + gcap + g], count = grp[1 + 2 * gcap + g];
    const int32_t *list = grp + 1 + 3 * gcap + start;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i0 = blockIdx.y * 16 + kDownRows * wave;
    const int nb = hidden >> 5;
    const uint8_t *w[kDownRows];
    const float *ws[kDownRows];
#pragma unroll
    for (int r = 0; r < kDownRows; r++) {
        const int i = min(i0 + r, dim - 1);
        w[r] = w2[e] + (int64_t)i * hidden;
        ws[r] = s2[e] + (int64_t)i * nb;
    }
    for (int p0 = 0; p0 < count; p0 += kMoePass) {
        const int np = min(kMoePass, count - p0);
        int pr[kMoePass];
        const int8_t *xq[kMoePass];
        const float *xsp[kMoePass];
#pragma unroll
        for (int j = 0; j < kMoePass; j++) {
            pr[j] = list[p0 + min(j, np - 1)];
            xq[j] = hq + (int64_t)pr[j] * hidden;
            xsp[j] = hs + (int64_t)pr[j] * nb;
        }
        float res[kMoePass][kDownRows];
        wave_rows_q8_multi<kDownRows, kMoePass>(w, ws, xq, xsp, np, hidden, res);
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < kMoePass; j++) {
                if (j >= np) break;
#pragma unroll
                for (int r = 0; r < kDownRows; r++)
                    if (i0 + r < dim) o[(int64_t)pr[j] * dim + i0 + r] = res[j][r];
            }
        }
    }
}

// The same W1/W3 and W2 products for inputs up to 2048 wide, eight lanes a
// row dot: a wave's rows are loaded once, up front (BPL blocks a lane), and
// the group's inputs are staged in LDS kExpTok at a time. moe_up8: wave w
// takes hidden rows 4w..4w+3 of the workgroup's 32 (W1 of row q in lanes
// 16q..16q+7, W3 in 16q+8..16q+15; the W3 dot moves beside the W1 dot by
// one DPP row shift). moe_down8: wave w takes W2 rows 8w..8w+7 of the
// workgroup's 32.
constexpr int kExpTok = 16;

__device__ __forceinline__ float row_shl8(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x108, 0xF, 0xF, false));
}

// LDS of moe_up8_kernel for inputs `dim` wide: kExpTok inputs' codes and
// scales (each region padded by a stripe of direct-to-LDS loads), h, the
// pass's pairs and their weights.
__host__ __device__ constexpr int up8_q_bytes(int dim) { return kExpTok * dim + 1024; }
__host__ __device__ constexpr int up8_s_bytes(int dim) { return kExpTok * (dim >> 5) * 4 + 256; }
__host__ __device__ constexpr int up8_lds(int dim) {
    return up8_q_bytes(dim) + up8_s_bytes(dim) + kExpTok * 32 * 4 + kExpTok * 8;
}

// ALL: the call's tokens (at most kExpTok) are staged in LDS at the start,
// every one of them, so the staging does not wait for the pair list; else
// each pass stages its own pairs' inputs. EX: the rows are exactly 8·BPL
// blocks, read in contiguous pieces (lane_row_load_pair), else whole
// blocks a lane. The group's rows, count and list are found with one load
// each (the grouping wrote the rows' addresses).
template <int BPL, bool ALL, bool EX>
__global__ __launch_bounds__(512) void moe_up8_kernel(const void *const *gptr, const int32_t *grp, int gcap,
                                                      const float *gwt, int k, const int8_t *qx, const float *xs,
                                                      int tokens, int dim, int hidden, int8_t *hq, float *hs,
                                                      int32_t *hsum) {
    extern __shared__ __align__(16) char ulds[];
    const int g = blockIdx.y;  // groups slowest: the live groups are dispatched first
    const int nb = dim >> 5;
    int8_t *sq = reinterpret_cast<int8_t *>(ulds);                                  // [kExpTok][dim] codes
    float *sxs = reinterpret_cast<float *>(ulds + up8_q_bytes(dim));                 // [kExpTok][nb] scales
    float *sh = reinterpret_cast<float *>(ulds + up8_q_bytes(dim) + up8_s_bytes(dim));  // [kExpTok][32] h
    int *spair = reinterpret_cast<int *>(sh + kExpTok * 32);                         // [kExpTok] pairs
    float *swt = reinterpret_cast<float *>(spair + kExpTok);                         // [kExpTok] their weights
    // independent loads first: the group count, this group's rows, start, count
    const int ngroups = grp[0];
    const uint8_t *w1 = static_cast<const uint8_t *>(gptr[6 * g]);
    const float *s1 = static_cast<const float *>(gptr[6 * g + 1]);
    const uint8_t *w3 = static_cast<const uint8_t *>(gptr[6 * g + 2]);
    const float *s3 = static_cast<const float *>(gptr[6 * g + 3]);
    const int start = grp[1 + gcap + g], count = grp[1 + 2 * gcap + g];
    if (g >= ngroups) return;  // uniform
    const int32_t *list = grp + 1 + 3 * gcap + start;
    const float *lwt = gwt + start;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = lane >> 3, rl = lane & 7, q = rg >> 1;
    const int j = blockIdx.x * 32 + 4 * wave + q;  // hidden is a multiple of 32
    const bool w3row = rg & 1;
    // the first pass's pairs and weights, then (ALL) every token's input,
    // then the rows: loads return in issue order
    int lp = 0;
    float lw = 0.0f;
    if (tid < min(kExpTok, count)) {
        lp = list[tid];
        lw = lwt[tid];
    }
    if (ALL) {
        // stripes of 64 pieces a wave; a last stripe's surplus lanes repeat
        // the last piece into the padding after the region
        const int nq = (tokens * dim) >> 4, ns = tokens * nb;
        for (int p0 = wave * 64; p0 < nq; p0 += 512)
            __builtin_amdgcn_global_load_lds(qx + 16 * min(p0 + lane, nq - 1), lds_ptr(sq + 16 * p0), 16, 0, 0);
        for (int p0 = wave * 64; p0 < ns; p0 += 512)
            __builtin_amdgcn_global_load_lds(xs + min(p0 + lane, ns - 1), lds_ptr(sxs + p0), 4, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    int4 c0[BPL], c1[BPL];
    float sw[BPL];
    if (EX)
        lane_row_load_pair<BPL>(c0, c1, sw, (w3row ? w3 : w1) + (int64_t)j * dim, (w3row ? s3 : s1) + (int64_t)j * nb,
                                nb, rl);
    else
        lane_row_load<BPL>(c0, c1, sw, (w3row ? w3 : w1) + (int64_t)j * dim, (w3row ? s3 : s1) + (int64_t)j * nb, nb,
                           rl);
    __builtin_amdgcn_sched_barrier(0);
    const int n16 = dim >> 4;
    for (int p0 = 0; p0 < count; p0 += kExpTok) {
        const int np = min(kExpTok, count - p0);
        if (p0 > 0 && tid < np) {
            lp = list[p0 + tid];
            lw = lwt[p0 + tid];
        }
        if (tid < np) {
            spair[tid] = lp;
            swt[tid] = lw;
        }
        if (ALL) __builtin_amdgcn_s_waitcnt(0);  // the direct-to-LDS loads (and the rows) have landed
        __syncthreads();
        if (!ALL) {
            for (int i = tid; i < np * n16; i += 512) {
                const int pi = i / n16, off = i - pi * n16;
                reinterpret_cast<int4 *>(sq)[i] =
                    reinterpret_cast<const int4 *>(qx + (int64_t)(spair[pi] / k) * dim)[off];
            }
            for (int i = tid; i < np * nb; i += 512) {
                const int pi = i / nb, b = i - pi * nb;
                sxs[i] = xs[(int64_t)(spair[pi] / k) * nb + b];
            }
            __syncthreads();
        }
        for (int pi = 0; pi < np; pi++) {
            const int u = ALL ? spair[pi] / k : pi;  // the input's place in LDS
            const float v = EX ? tree8_pair(lane_running_sum_pair<BPL, true>(c0, c1, sw, sq + u * dim, sxs + u * nb, nb, rl))
                               : tree8(lane_running_sum<BPL>(c0, c1, sw, sq + u * dim, sxs + u * nb, nb, rl));
            const float v3 = row_shl8(v);  // lane 16q: the W3 dot of row q
            if ((lane & 15) == 0) sh[pi * 32 + 4 * wave + q] = swt[pi] * silu_mul(v, v3);
        }
        __syncthreads();
        // each pair's block of h: wave w takes pairs w, w+8, ...; lanes 0-7
        // four values each (every lane of the wave calls the quantizer)
        for (int pi = wave; pi < np; pi += 8) {
            const float4 v4 = reinterpret_cast<const float4 *>(sh + pi * 32)[min(lane, 7)];
            float d;
            int cs;
            const uint32_t pk = quantize_group(v4.x, v4.y, v4.z, v4.w, d, cs);
            const int64_t base = (int64_t)spair[pi] * hidden + blockIdx.x * 32;
            if (lane < 8) {
                reinterpret_cast<uint32_t *>(hq + base)[lane] = pk;
                if (lane == 0) {
                    hs[base >> 5] = d;
                    hsum[base >> 5] = cs;
                }
            }
        }
        __syncthreads();
    }
}

// moe_up1_kernel's LDS: the normed input's codes, scales and code sums,
// then per expert (E rounded up to 4) a float, a 64-bit key and a rank, the
// norm's transposed x, and the experts' W1/W3 row and scale pointers.
struct Up1Lds {
    int sxs, sxsum, sp, skey, srank, sn, stab, bytes;
};
__host__ __device__ inline Up1Lds up1_lds(int dim, int experts) {
    Up1Lds l;
    const int nb = dim >> 5, ep = (experts + 3) & ~3;
    l.sxs = dim;
    l.sxsum = l.sxs + 4 * nb;
    l.sp = (l.sxsum + 4 * nb + 15) & ~15;
    l.skey = l.sp + 4 * ep;
    l.srank = l.skey + 8 * (ep > 128 ? ep : 128);  // (up to 128 experts: the ranks read 128 keys)
    l.sn = (l.srank + 4 * ep + 15) & ~15;
    l.stab = l.sn + 32 * ((((dim >> 5) + 3) & ~3) + 4) * 4;
    l.bytes = l.stab + 8 * 4 * experts;
    return l;
}
constexpr int kUp1MaxExperts = 512;

// route_wave's softmax of one token by one wave (every lane calls it): lg
// holds the logits of experts lane + 64j; the probabilities go to sp and
// each expert's key (route_key) to skey. Every lane runs the one sequential
// sum (the wave's LDS writes precede its reads), so all get the same inv.
template <int LPER>
__device__ __forceinline__ void up1_softmax(const float (&lg)[LPER], int experts, float *sp, unsigned long long *skey) {
    const int lane = threadIdx.x & 63;
    float m = lg[0];
#pragma unroll
    for (int j = 0; j < LPER; j++)
        if (lane + 64 * j < experts) m = gomax(m, lg[j]);
    m = wave_gomax(m);
#pragma unroll
    for (int j = 0; j < LPER; j++)
        if (lane + 64 * j < experts) sp[lane + 64 * j] = exp32(lg[j] - m);
    const float inv = recip32(lds_chain_sum(sp, experts, 0.0f));
#pragma unroll
    for (int j = 0; j < LPER; j++) {
        const int e = lane + 64 * j;
        if (e < experts) {
            const float pv = sp[e] * inv;
            sp[e] = pv;
            skey[e] = route_key(pv, e);
        }
    }
}

// The stable top-k as ranks over a 512-thread workgroup: each expert's
// count of larger keys (keys are distinct, so the k largest have ranks
// 0..k-1, in the order route_wave's rounds pick them), TPE threads an
// expert, each counting over a slice of the keys (pairs read 16 bytes at a
// time, four reads in flight), summed into srank (cleared before) by LDS
// atomics. Every thread calls it; skey and srank in LDS.
__device__ __forceinline__ void expert_ranks(const unsigned long long *skey, int *srank, int experts) {
    const int tid = threadIdx.x;
    int ep = 1;
    while (ep < experts) ep <<= 1;
    const int tpe = max(1, 512 / ep);
    const int slice = ((experts + tpe - 1) / tpe + 1) & ~1;  // even: 16-byte pairs
    const int e = tid / tpe, part = tid - e * tpe;
    if (e >= experts) return;
    const unsigned long long ke = skey[e];
    int c = 0, q = part * slice;
    const int hi = min(experts, q + slice);
    for (; q + 8 <= hi; q += 8) {
        const ulonglong2 *p2 = reinterpret_cast<const ulonglong2 *>(skey + q);
        const ulonglong2 a = p2[0], b = p2[1], u = p2[2], v = p2[3];
        c += (a.x > ke) + (a.y > ke) + (b.x > ke) + (b.y > ke) + (u.x > ke) + (u.y > ke) + (v.x > ke) + (v.y > ke);
    }
    for (; q < hi; q++) c += skey[q] > ke ? 1 : 0;
    if (c) atomicAdd(&srank[e], c);
}

// One token's W1/W3 rows with the ffn RMSNorm and the routing folded in.
// Every workgroup forms RMSNorm_ffn(x)'s Q8_0 input in LDS and routes the
// token itself (every workgroup gets the same selection); workgroup (g, b)
// then takes the g-th selected expert by ascending index and its hidden
// rows 32b .. 32b+31 (W1 and W3 of each: eight row dots a wave, eight lanes
// a row); h as moe_up8_kernel's. Workgroup (0, 0) also writes the
// selection, the weights and the grouping (one pair a group) for the W2
// products and the sum. The routing's steps are route_wave's, spread over
// the workgroup: wave 1 the softmax while wave 0 runs the norm's Dot32
// chain, then the stable top-k as ranks (each expert's count of larger
// keys; keys are distinct) by all waves, the weights by wave 0. The
// experts' row pointers are staged in LDS while the token is routed.
// (Computing the router's logits in every workgroup instead, from its rows
// in L2, was measured slower: issuing 1.125·E·dim bytes of row loads per
// workgroup took longer than the router's own launch.)
template <int BPL>
__global__ __launch_bounds__(512) void moe_up1_kernel(const float *x, const float *norm_w, float recip_n, float eps,
                                                      const float *logits, int experts, int k,
                                                      const uint8_t *const *w1, const float *const *s1,
                                                      const uint8_t *const *w3, const float *const *s3,
                                                      const uint8_t *const *w2, const float *const *s2, int dim,
                                                      int hidden, int32_t *sel, float *wsel, int gcap, int32_t *grp,
                                                      const void **gptr, int8_t *hq, float *hs, int32_t *hsum) {
    extern __shared__ __align__(16) char ulds[];
    __shared__ float bcast, s_w;
    __shared__ int s_e, s_slot;
    __shared__ int ssel[kMoeMaxK];
    __shared__ __align__(16) float sh[32];
    const Up1Lds L = up1_lds(dim, experts);
    const int nb = dim >> 5;
    int8_t *sq = reinterpret_cast<int8_t *>(ulds);                                  // [dim] codes
    float *sxs = reinterpret_cast<float *>(ulds + L.sxs);                          // [nb] scales
    int32_t *sxsum = reinterpret_cast<int32_t *>(ulds + L.sxsum);                  // [nb] code sums
    float *sp = reinterpret_cast<float *>(ulds + L.sp);                            // [experts] probabilities
    unsigned long long *skey = reinterpret_cast<unsigned long long *>(ulds + L.skey);
    int *srank = reinterpret_cast<int *>(ulds + L.srank);
    float *sn = reinterpret_cast<float *>(ulds + L.sn);                            // the norm's transposed x
    const void **stab = reinterpret_cast<const void **>(ulds + L.stab);            // [4][experts] row pointers
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = lane >> 3, rl = lane & 7;
    // loads: x and the norm weights (a group of four a thread), the logits
    // (wave 1), the row pointer tables
    const int ng = dim >> 2;
    const int g4 = min(tid, ng - 1);
    const float4 xv = reinterpret_cast<const float4 *>(x)[g4];
    const float4 wv = reinterpret_cast<const float4 *>(norm_w)[g4];
    constexpr int kLPer = kUp1MaxExperts / 64;
    float lg[kLPer];
    if (wave == 1) {
#pragma unroll
        for (int j = 0; j < kLPer; j++) lg[j] = logits[min(lane + 64 * j, experts - 1)];
    }
    for (int t = tid; t < 4 * experts; t += 512) {
        const int tab = t / experts, e = t - tab * experts;
        stab[t] = tab == 0 ? (const void *)w1[e] : tab == 1 ? (const void *)s1[e] : tab == 2 ? (const void *)w3[e]
                                                                                           : (const void *)s3[e];
    }
    // x transposed for Dot32 (xt[j·pitch + m] = x_{j+32m}); ranks cleared
    const int steps = dim >> 5, pitch = ((steps + 3) & ~3) + 4;
    if (tid < ng) {
        const int i = 4 * tid;
        float *d = sn + (i & 31) * pitch + (i >> 5);
        d[0] = xv.x;
        d[pitch] = xv.y;
        d[2 * pitch] = xv.z;
        d[3 * pitch] = xv.w;
    }
    for (int e = tid; e < experts; e += 512) srank[e] = 0;
    __syncthreads();
    if (wave == 0) {
        // RMSNorm (model.go:632-638): ss = Dot32(x, x)·recip_n + eps
        const float sq32 = lane < 32 ? lds_dot32_self_t(sn, pitch, steps, lane) : 0.0f;
        const float dot = dot32_reduce(sq32);
        if (lane == 0) bcast = rsqrt32((dot * recip_n) + eps);
    } else if (wave == 1) {
        up1_softmax<kLPer>(lg, experts, sp, skey);
    }
    __syncthreads();
    {
        // the normed input's Q8_0 (quant.go:34-53): out_i = w_i·(r·x_i)
        const float r = bcast;
        float d;
        int cs;
        const uint32_t pk = quantize_group(wv.x * (r * xv.x), wv.y * (r * xv.y), wv.z * (r * xv.z),
                                           wv.w * (r * xv.w), d, cs);
        if (tid < ng) {
            reinterpret_cast<uint32_t *>(sq)[tid] = pk;
            if ((tid & 7) == 0) {
                sxs[tid >> 3] = d;
                sxsum[tid >> 3] = cs;
            }
        }
    }
    __syncthreads();
    expert_ranks(skey, srank, experts);
    __syncthreads();
    for (int e = tid; e < experts; e += 512)
        if (srank[e] < k) ssel[srank[e]] = e;
    __syncthreads();
    const bool lead = blockIdx.x == 0 && blockIdx.y == 0;
    if (wave == 0 && lane < k) {
        const int mine = ssel[lane];
        const float ps = sp[mine];
        // the weights (route_wave's): the selected probabilities' sum in
        // selection order from +0, times its Recip32
        float sum = 0.0f;
        for (int r = 0; r < k; r++) sum += __shfl(ps, r);
        const float wt = ps * recip32(sum);
        int r = 0;  // place among the selection by ascending index (the experts are distinct)
        for (int q = 0; q < k; q++) r += ssel[q] < mine;
        if (r == (int)blockIdx.x) {
            s_e = mine;
            s_w = wt;
            s_slot = lane;
        }
        if (lead) {
            sel[lane] = mine;
            wsel[lane] = wt;
            grp[1 + r] = mine;
            grp[1 + gcap + r] = r;
            grp[1 + 2 * gcap + r] = 1;
            grp[1 + 3 * gcap + r] = lane;  // pair (token 0, slot lane)
            gptr[6 * r + 4] = w2[mine];    // the W2 rows the sum's launch reads
            gptr[6 * r + 5] = s2[mine];
            if (lane == 0) grp[0] = k;
        }
    }
    __syncthreads();
    const int e = s_e;
    const int q = rg >> 1;
    const int j = blockIdx.y * 32 + 4 * wave + q;
    const bool w3row = rg & 1;
    const uint8_t *wrow = static_cast<const uint8_t *>(stab[(w3row ? 2 : 0) * experts + e]);
    const float *srow = static_cast<const float *>(stab[(w3row ? 3 : 1) * experts + e]);
    int4 c0[BPL], c1[BPL];
    float sw[BPL];
    lane_row_load_pair<BPL>(c0, c1, sw, wrow + (int64_t)j * dim, srow + (int64_t)j * nb, nb, rl);
    const float v = tree8_pair(lane_running_sum_pair<BPL>(c0, c1, sw, sq, sxs, nb, rl));
    const float v3 = row_shl8(v);  // lane 16q: the W3 dot of row q
    if ((lane & 15) == 0) sh[4 * wave + q] = s_w * silu_mul(v, v3);
    __syncthreads();
    if (wave == 0) {
        const float4 v4 = reinterpret_cast<const float4 *>(sh)[min(lane, 7)];
        float d;
        int cs;
        const uint32_t pk = quantize_group(v4.x, v4.y, v4.z, v4.w, d, cs);
        const int64_t base = (int64_t)s_slot * hidden + blockIdx.y * 32;
        if (lane < 8) {
            reinterpret_cast<uint32_t *>(hq + base)[lane] = pk;
            if (lane == 0) {
                hs[base >> 5] = d;
                hsum[base >> 5] = cs;
            }
        }
    }
}

// EX: the W2 rows are exactly 8·BPL blocks (unclamped running sums).
template <int BPL, bool EX>
__global__ __launch_bounds__(256) void moe_down8_kernel(const void *const *gptr, const int32_t *grp, int gcap,
                                                        const int8_t *hq, const float *hs, int dim, int hidden,
                                                        float *o) {
    extern __shared__ __align__(16) char dlds[];
    const int g = blockIdx.y;  // groups slowest: the live groups are dispatched first
    // independent loads first: the group count, this group's rows, start, count
    const int ngroups = grp[0];
    const uint8_t *w2 = static_cast<const uint8_t *>(gptr[6 * g + 4]);
    const float *s2 = static_cast<const float *>(gptr[6 * g + 5]);
    const int start = grp[1 + gcap + g], count = grp[1 + 2 * gcap + g];
    if (g >= ngroups) return;  // uniform
    const int32_t *list = grp + 1 + 3 * gcap + start;
    const int nb = hidden >> 5;
    int8_t *sq = reinterpret_cast<int8_t *>(dlds);                        // [kExpTok][hidden] codes
    float *sxs = reinterpret_cast<float *>(dlds + kExpTok * hidden);       // [kExpTok][nb] scales
    int *spair = reinterpret_cast<int *>(sxs + kExpTok * nb);              // [kExpTok] pairs
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rg = lane >> 3, rl = lane & 7;
    const int i = blockIdx.x * 32 + 8 * wave + rg;
    // the first pass's pairs, requested before the rows (loads return in
    // issue order)
    int lp = 0;
    if (tid < min(kExpTok, count)) lp = list[tid];
    __builtin_amdgcn_sched_barrier(0);
    int4 c0[BPL], c1[BPL];
    float sw[BPL];
    lane_row_load_pair<BPL>(c0, c1, sw, w2 + (int64_t)min(i, dim - 1) * hidden, s2 + (int64_t)min(i, dim - 1) * nb, nb,
                       rl);
    __builtin_amdgcn_sched_barrier(0);
    const int n16 = hidden >> 4;
    for (int p0 = 0; p0 < count; p0 += kExpTok) {
        const int np = min(kExpTok, count - p0);
        if (p0 > 0 && tid < np) lp = list[p0 + tid];
        if (tid < np) spair[tid] = lp;
        __syncthreads();
        for (int u = tid; u < np * n16; u += 256) {
            const int pi = u / n16, off = u - pi * n16;
            reinterpret_cast<int4 *>(sq)[u] = reinterpret_cast<const int4 *>(hq + (int64_t)spair[pi] * hidden)[off];
        }
        for (int u = tid; u < np * nb; u += 256) {
            const int pi = u / nb, b = u - pi * nb;
            sxs[u] = hs[(int64_t)spair[pi] * nb + b];
        }
        __syncthreads();
        for (int pi = 0; pi < np; pi++) {
            const float v =
                tree8_pair(lane_running_sum_pair<BPL, EX>(c0, c1, sw, sq + pi * hidden, sxs + pi * nb, nb, rl));
            if (rl == 0 && i < dim) o[(int64_t)spair[pi] * dim + i] = v;
        }
        __syncthreads();
    }
}

// One token's W2 rows and the sum in one launch: workgroup b takes output
// rows R·b .. R·b+R-1 (R = 64 / k) of every selected expert (group of eight
// lanes gi: expert group gi / R, row gi mod R; h read from global), then
// lane r adds row r's k products in ascending expert order from +0 (the
// grouping's order) into y, out = y or Canonical(out + y). The same bits as
// moe_down8_kernel followed by moe_combine_kernel.
template <int BPL>
__global__ __launch_bounds__(512) void moe_down1_kernel(const void *const *gptr, const int32_t *grp, int gcap, int k,
                                                        const int8_t *hq, const float *hs, int dim, int hidden,
                                                        float *out, int residual) {
    __shared__ float sv[64];
    const int R = 64 / k;
    const int tid = threadIdx.x, gi = tid >> 3, rl = tid & 7;
    const int g = min(gi / R, k - 1), r = gi - (gi / R) * R;
    const int i = blockIdx.x * R + r;
    const int nb = hidden >> 5;
    // the one-token grouping (moe_up1_kernel's): group g's pair is list[g],
    // its W2 rows at gptr[6g + 4], [6g + 5]
    const uint8_t *w2 = static_cast<const uint8_t *>(gptr[6 * g + 4]);
    const float *s2 = static_cast<const float *>(gptr[6 * g + 5]);
    const int p = grp[1 + 3 * gcap + g];
    int4 c0[BPL], c1[BPL];
    float sw[BPL];
    lane_row_load_pair<BPL>(c0, c1, sw, w2 + (int64_t)min(i, dim - 1) * hidden, s2 + (int64_t)min(i, dim - 1) * nb, nb, rl);
    const float v = tree8_pair(lane_running_sum_pair<BPL>(c0, c1, sw, hq + (int64_t)p * hidden, hs + (int64_t)p * nb, nb, rl));
    if (rl == 0 && gi < k * R) sv[gi] = v;
    __syncthreads();
    if (tid < R && blockIdx.x * R + tid < dim) {
        float y = 0.0f;
        for (int q = 0; q < k; q++) y += sv[q * R + tid];
        float *dst = out + blockIdx.x * R + tid;
        *dst = residual ? canonical(*dst + y) : y;
    }
}

// ---------------------------------------------------------------------------
// One token's whole feed-forward in one launch (a decode step): the router
// product with the RMSNorm, the routing, each selected expert's W1/W3 rows
// and W2 rows, and the ascending-order sum into the residual. The bits are
// those of the router's launch (launch_fused with the norm prologue),
// moe_up1_kernel and moe_down1_kernel. Workgroups of eight waves, in grid
// order:
//  * nr router workgroups of eight router rows (one a wave; lane b holds
//    the row's block b, inputs up to 2048 wide): RMSNorm(x)'s Q8_0 input in
//    LDS, each row's block terms float32(sum_b)·float32(ws_b·xs_b) in LDS by
//    running sum b mod 8, eight lanes adding them in block order from +0,
//    the tree ((0+1)+(2+3))+((4+5)+(6+7)) (MatVecQ8, quant.go:158-180).
//    Workgroup 0 then collects the logits and routes the token
//    (moe_up1_kernel's steps, spread over the workgroup).
//  * nu up workgroups (place g, block hb of 32 hidden rows): the normed
//    input, the wait for the selection, then the g-th selected expert's W1
//    and W3 rows (four hidden rows a wave, eight lanes a row dot) and h as
//    moe_up1_kernel's: one Q8_0 block, put at place g (tag_put_q8).
//  * nd down workgroups of R = 64/k output rows of every selected expert:
//    the W2 rows requested once the selection is seen, every block of h
//    collected into LDS (tag_get_q8), the row dots, and lane r adding row
//    r's k products by ascending expert from +0 into y; out = y or
//    Canonical(out + y).
// Every hand-off is a tagged word (rk_sync.h), each workgroup keeping one
// count word of its own (a layer's grid is fixed). The logits are one word
// each; the selection is written by ascending expert index into every
// XCD's line (the experts first, then their weights, which only the up
// rows' ends need); h's blocks are tag_put_q8's six words. The words are
// the layer's own (ffn1_sync_layout): tags count that layer's launches.
// A workgroup waits only for workgroups before it in the grid, which are
// dispatched before it, so the launch always drains. Every wait is bounded
// by the device clock (kSyncTimeout); one that gives up sets *err and goes
// on with what memory holds, expert indices clamped into range.
constexpr int kFfn1MaxK = 16;         // the selection's experts, then their weights, in an XCD's line
constexpr int kFfn1LineWords = 2 * kFfn1MaxK;
constexpr int kFfn1MaxExperts = 512;  // eight a lane of the collecting wave
constexpr int kFfn1MaxCols = 2048;    // one input block a lane of a router row
constexpr int kFfn1MaxHidden = 2048;  // eight W2 blocks a lane

struct Ffn1Args {
    const float *x, *norm_w;
    float recip_n, eps;
    const uint8_t *rw;  // the router [experts][dim] and its scales
    const float *rws;
    const uint8_t *const *w1;
    const uint8_t *const *w3;
    const uint8_t *const *w2;
    const float *const *s1;
    const float *const *s3;
    const float *const *s2;
    int experts, k, dim, hidden;
    int32_t *sel;  // [k] the selection in selection order, and its weights
    float *wsel;
    float *out;
    int residual;
    // the layer's hand-off words (ffn1_sync_layout), zero when made
    unsigned long long *lines;  // [8][kFfn1LineWords] the selection, a line per XCD
    unsigned long long *lw;     // [experts] the tagged logits
    unsigned long long *hw;     // [k][hidden/32][6] h's Q8_0 blocks as tagged words (tag_put_q8)
    unsigned long long *cnt;    // [nr + nu + nd] each workgroup's count of its launches
    unsigned long long *err;
    int nr, nu, nd;  // router, up and down workgroups
};

// The hand-off words of one layer: the selection lines, the tagged logits,
// h's tagged blocks and every workgroup's launch count (each in whole
// 128-byte lines).
struct Ffn1Sync {
    int64_t lines, lw, hw, cnt, words;
};
inline Ffn1Sync ffn1_sync_layout(int dim, int experts, int k, int hidden) {
    auto al = [](int64_t w) { return (w + 15) & ~(int64_t)15; };
    const int64_t nr = (experts + 7) / 8, nu = (int64_t)k * (hidden / 32), nd = (dim + 64 / k - 1) / (64 / k);
    Ffn1Sync l;
    l.lines = 0;
    l.lw = 8 * kFfn1LineWords;
    l.hw = l.lw + al(experts);
    l.cnt = l.hw + al(6 * nu);
    l.words = l.cnt + al(nr + nu + nd);
    return l;
}

// LDS (bytes): the normed input's codes and scales and the norm's
// transposed x, then each role's own: the router's terms [8][64], the
// probabilities, keys and ranks [experts]; the up rows' pointer tables
// [4][experts] and h [32]; the down rows' tables [2][experts], h
// [k][hidden], its scales, and the row dots [64].
struct Ffn1Lds {
    int sxs, sn, role, sp, skey, srank, hq, hs, sv, bytes;
};
__host__ __device__ inline Ffn1Lds ffn1_lds(int dim, int experts, int k, int hidden) {
    Ffn1Lds l;
    const int nb = dim >> 5, pitch = ((nb + 3) & ~3) + 4, ep = (experts + 3) & ~3;
    l.sxs = (dim + 15) & ~15;
    l.sn = (l.sxs + 4 * nb + 15) & ~15;
    l.role = (l.sn + 4 * 32 * pitch + 15) & ~15;
    l.sp = l.role + 8 * 64 * 4;
    l.skey = l.sp + 4 * ep;
    l.srank = l.skey + 8 * ep;
    const int router = l.srank + 4 * ep;
    const int up = l.role + 8 * 4 * experts + 32 * 4;
    l.hq = l.role + 8 * 2 * experts;
    l.hs = l.hq + ((k * hidden + 15) & ~15);
    l.sv = l.hs + ((4 * k * (hidden >> 5) + 15) & ~15);
    const int down = l.sv + 64 * 4;
    l.bytes = router > up ? (router > down ? router : down) : (up > down ? up : down);
    return l;
}

// RMSNorm(x) (model.go:632-638) and its Q8_0 form (quant.go:34-53) into
// LDS by a 512-thread workgroup, thread t holding x's and the weights'
// group t (clamped): x transposed into sn, Dot32 by wave 0, then
// quantize_group (moe_up1_kernel's steps). Ends with a barrier.
__device__ __forceinline__ void ffn1_norm_quant(float4 xv, float4 wv, int dim, float recip_n, float eps, int8_t *sq,
                                                float *sxs, float *sn, float *bcast) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int ng = dim >> 2, steps = dim >> 5, pitch = ((steps + 3) & ~3) + 4;
    if (tid < ng) {
        const int i = 4 * tid;
        float *d = sn + (i & 31) * pitch + (i >> 5);
        d[0] = xv.x;
        d[pitch] = xv.y;
        d[2 * pitch] = xv.z;
        d[3 * pitch] = xv.w;
    }
    __syncthreads();
    if (tid < 64) {
        const float s = lane < 32 ? lds_dot32_self_t(sn, pitch, steps, lane) : 0.0f;
        const float dot = dot32_reduce(s);
        if (lane == 0) *bcast = rsqrt32((dot * recip_n) + eps);
    }
    __syncthreads();
    const float r = *bcast;
    float d;
    int cs;
    const uint32_t pk =
        quantize_group(wv.x * (r * xv.x), wv.y * (r * xv.y), wv.z * (r * xv.z), wv.w * (r * xv.w), d, cs);
    if (tid < ng) {
        reinterpret_cast<uint32_t *>(sq)[tid] = pk;
        if ((tid & 7) == 0) sxs[tid >> 3] = d;
    }
    __syncthreads();
}


// The routing of launch n by router workgroup 0 (every thread calls it):
// wave 0 polls the tagged logits until all E carry the launch's tag, then
// the softmax (up1_softmax: Go max, Exp32, one sequential sum, Recip32) and
// each expert's key, the stable top-k as ranks (expert_ranks), the weights
// p·Recip32(Σ p) with the sum in selection order from +0; sel/wsel in
// selection order and the tagged words by ascending expert.
template <int PER>
__device__ void ffn1_route(const Ffn1Args &a, uint32_t tag, float *sp, unsigned long long *skey, int *srank,
                           int *ssel) {
    const int tid = threadIdx.x, lane = tid & 63, E = a.experts, k = a.k;
    if (PER > 2)
        for (int e = tid; e < E; e += 512) srank[e] = 0;
    if (tid < 64) {
        float lg[PER];
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        bool ok = false;
        for (int i = 0; i < (1 << 24); i++) {
            bool mine = true;
#pragma unroll
            for (int j = 0; j < PER; j++) {
                if (64 * j < E) {  // uniform
                    const unsigned long long v =
                        __hip_atomic_load(a.lw + min(lane + 64 * j, E - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    lg[j] = u2f((uint32_t)v);
                    mine = mine && (uint32_t)(v >> 48) == tag;
                } else {
                    lg[j] = 0.0f;
                }
            }
            if (__all(mine)) {
                ok = true;
                break;
            }
            if (__builtin_amdgcn_s_memrealtime() - t0 > kSyncTimeout) break;
            __builtin_amdgcn_s_sleep(1);
        }
        if (!ok && lane == 0) __hip_atomic_store(a.err, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        float m = lg[0];
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (lane + 64 * j < E) m = gomax(m, lg[j]);
        m = wave_gomax(m);
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (lane + 64 * j < E) sp[lane + 64 * j] = exp32(lg[j] - m);
        const float inv = recip32(lds_chain_sum(sp, E, 0.0f));
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int e = lane + 64 * j;
            if (e < E) {
                const float pv = sp[e] * inv;
                sp[e] = pv;
                skey[e] = route_key(pv, e);
            }
        }
    }
    __syncthreads();
    if (PER == 2) {
        // up to 128 experts: thread t counts the larger keys of expert t/4
        // among key pairs 8q + 2(t mod 4), q < 16 (the quad's four reads
        // of a step in distinct banks); the quad's counts summed by DPP
        const int e = tid >> 2, part = tid & 3;
        const unsigned long long ke = skey[min(e, E - 1)];
        const ulonglong2 *p2 = reinterpret_cast<const ulonglong2 *>(skey) + part;
        int c = 0;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const ulonglong2 v = p2[4 * q];
            const int i0 = 8 * q + 2 * part;
            c += ((i0 < E) & (v.x > ke)) + ((i0 + 1 < E) & (v.y > ke));
        }
        c += dpp_x1(c);
        c += dpp_x2(c);
        if (part == 0 && e < E && c < k) ssel[c] = e;
    } else {
        expert_ranks(skey, srank, E);
        __syncthreads();
        for (int e = tid; e < E; e += 512)
            if (srank[e] < k) ssel[srank[e]] = e;
    }
    __syncthreads();
    if (tid < 64) {
        const int mine = ssel[min(lane, k - 1)];
        int place = 0;  // among the selection by ascending index (the experts are distinct)
        for (int q = 0; q < k; q++) place += ssel[q] < mine ? 1 : 0;
        // the experts first: the up and down workgroups request their rows
        // on them; the weights are needed only after the up rows' dots
        if (lane < k) {
            const unsigned long long word = ((unsigned long long)tag << 48) | (unsigned long long)(mine & 0xFFFF);
#pragma unroll
            for (int xcd = 0; xcd < 8; xcd++)
                __hip_atomic_store(a.lines + kFfn1LineWords * xcd + place, word, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        const float ps = sp[mine];
        float sum = 0.0f;
        for (int r = 0; r < k; r++) sum += __shfl(ps, r);
        const float wt = ps * recip32(sum);
        if (lane < k) {
            const unsigned long long word = ((unsigned long long)tag << 48) | (unsigned long long)f2u(wt);
#pragma unroll
            for (int xcd = 0; xcd < 8; xcd++)
                __hip_atomic_store(a.lines + kFfn1LineWords * xcd + kFfn1MaxK + place, word, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            a.sel[lane] = mine;
            a.wsel[lane] = wt;
        }
    }
}

// The waits for the selection of launch `tag`, by one wave (every lane
// calls them): polls of its XCD's line until words off .. off+k-1 all carry
// the tag; the experts (clamped) into s_e, or the weights into s_w.
__device__ void ffn1_wait_line(const Ffn1Args &a, uint32_t tag, int off, int *s_e, float *s_w) {
    const int lane = threadIdx.x & 63, k = a.k;
    const unsigned long long *line = a.lines + kFfn1LineWords * (blockIdx.x & 7) + off;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    unsigned long long v = 0;
    bool ok = false;
    for (int i = 0; i < (1 << 24); i++) {
        v = lane < k ? __hip_atomic_load(line + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : ((unsigned long long)tag << 48);
        if (__all((uint32_t)(v >> 48) == tag)) {
            ok = true;
            break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t0 > kSyncTimeout) break;
        __builtin_amdgcn_s_sleep(1);
    }
    if (!ok && lane == 0) __hip_atomic_store(a.err, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (lane < k) {
        if (s_e) s_e[lane] = min((int)(v & 0xFFFF), a.experts - 1);
        if (s_w) s_w[lane] = u2f((uint32_t)v);
    }
}

// EX: the up rows are exactly 8·BU blocks and the down rows 8·BD (the
// running sums' input offsets need no clamp).
template <int BU, int BD, bool EX>
__global__ __launch_bounds__(512) void moe_ffn1_kernel(Ffn1Args a) {
    extern __shared__ __align__(16) char flds[];
    __shared__ float bcast;
    __shared__ int s_e[kFfn1MaxK];
    __shared__ float s_w[kFfn1MaxK];
    __shared__ int s_to;
    const int dim = a.dim, nb = dim >> 5, E = a.experts, k = a.k, H = a.hidden, nhb = H >> 5;
    const Ffn1Lds L = ffn1_lds(dim, E, k, H);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bid = blockIdx.x;
    int8_t *sq = reinterpret_cast<int8_t *>(flds);
    float *sxs = reinterpret_cast<float *>(flds + L.sxs);
    float *sn = reinterpret_cast<float *>(flds + L.sn);
    const void **stab = reinterpret_cast<const void **>(flds + L.role);
    const unsigned long long cnt0 = a.cnt[bid];  // this workgroup's own count (a layer's grid is fixed)

    if (bid >= a.nr + a.nu) {
        // ---- down: output rows R·di .. R·di+R-1 of every selected expert;
        // group of eight lanes gi: place gi / R, row gi mod R ----
        const int di = bid - a.nr - a.nu, R = 64 / k;
        const int gi = tid >> 3, rl = tid & 7;
        const int g = min(gi / R, k - 1), r = gi - (gi / R) * R;
        const int64_t i = min(di * R + r, dim - 1);
        int8_t *shq = reinterpret_cast<int8_t *>(flds + L.hq);
        float *shs = reinterpret_cast<float *>(flds + L.hs);
        float *sv = reinterpret_cast<float *>(flds + L.sv);
        for (int t = tid; t < 2 * E; t += 512) stab[t] = t < E ? (const void *)a.w2[t] : (const void *)a.s2[t - E];
        __syncthreads();
        const uint32_t tag = tag_of(tag_take(cnt0, a.cnt + bid, 1));
        if (wave == 0) ffn1_wait_line(a, tag, 0, s_e, nullptr);
        __syncthreads();
        const int e = s_e[g];
        int4 c0[BD], c1[BD];
        float sw[BD];
        lane_row_load_pair<BD>(c0, c1, sw, static_cast<const uint8_t *>(stab[e]) + i * H,
                          static_cast<const float *>(stab[E + e]) + i * nhb, nhb, rl);
        tag_get_q8<512>(a.hw, k * nhb, tag, shq, shs, a.err, &s_to);
        const float v = tree8_pair(lane_running_sum_pair<BD, EX>(c0, c1, sw, shq + g * H, shs + g * nhb, nhb, rl));
        if (rl == 0 && gi < k * R) sv[gi] = v;
        __syncthreads();
        if (tid < R && di * R + tid < dim) {
            float y = 0.0f;
            for (int q = 0; q < k; q++) y += sv[q * R + tid];
            float *dst = a.out + di * R + tid;
            *dst = a.residual ? canonical(*dst + y) : y;
        }
        return;
    }

    // router and up workgroups: x and the norm weights, a group of four a thread
    const int g4 = min(tid, (dim >> 2) - 1);
    const float4 xv = reinterpret_cast<const float4 *>(a.x)[g4];
    const float4 wv = reinterpret_cast<const float4 *>(a.norm_w)[g4];

    if (bid < a.nr) {
        // ---- router rows 8·bid + wave ----
        const int row = bid * 8 + wave;
        const int64_t rr = min(row, E - 1);
        const int b = min(lane, nb - 1);
        const uint8_t *rp = a.rw + rr * dim + 32 * b;
        const int4 c0 = load_stream16_g(rp), c1 = load_stream16_g(rp + 16);
        const float sw = loadf_g(a.rws + rr * nb + b);
        ffn1_norm_quant(xv, wv, dim, a.recip_n, a.eps, sq, sxs, sn, &bcast);
        const uint32_t tag = tag_of(tag_take(cnt0, a.cnt + bid, 1));
        const int4 *xp = reinterpret_cast<const int4 *>(sq + 32 * b);
        const int sm = dot16(c1, xp[1], dot16(c0, xp[0], 0));
        const float t = (float)sm * (sw * sxs[b]);
        float *tw = reinterpret_cast<float *>(flds + L.role) + wave * 64;  // [running sum][b / 8]
        if (lane < nb) tw[(lane & 7) * 8 + (lane >> 3)] = t;
        __syncthreads();
        float acc = 0.0f;
        if (lane < 8) {
            const float *p = tw + lane * 8;
            const int cnt = lane < nb ? (nb - lane + 7) >> 3 : 0;
            for (int m = 0; m < cnt; m++) acc += p[m];
        }
        acc = tree8(acc);
        if (lane == 0 && row < E)
            __hip_atomic_store(a.lw + row, ((unsigned long long)tag << 48) | (unsigned long long)f2u(acc),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (bid == 0) {
            float *sp = reinterpret_cast<float *>(flds + L.sp);
            unsigned long long *skey = reinterpret_cast<unsigned long long *>(flds + L.skey);
            int *srank = reinterpret_cast<int *>(flds + L.srank);
            if (E <= 128)
                ffn1_route<2>(a, tag, sp, skey, srank, s_e);
            else
                ffn1_route<kFfn1MaxExperts / 64>(a, tag, sp, skey, srank, s_e);
        }
        return;
    }

    // ---- up: place g, hidden rows 32·hb .. 32·hb+31 (wave w rows 4w..4w+3:
    // W1 of row q in lanes 16q..16q+7, W3 in 16q+8..16q+15) ----
    const int ui = bid - a.nr, g = ui / nhb, hb = ui - g * nhb;
    float *sh = reinterpret_cast<float *>(flds + L.role + 8 * 4 * E);
    for (int t = tid; t < 4 * E; t += 512) {
        const int tab = t / E, e = t - tab * E;
        stab[t] = tab == 0 ? (const void *)a.w1[e] : tab == 1 ? (const void *)a.s1[e] : tab == 2 ? (const void *)a.w3[e]
                                                                                            : (const void *)a.s3[e];
    }
    ffn1_norm_quant(xv, wv, dim, a.recip_n, a.eps, sq, sxs, sn, &bcast);
    const uint32_t tag = tag_of(tag_take(cnt0, a.cnt + bid, 1));
    if (wave == 0) ffn1_wait_line(a, tag, 0, s_e, nullptr);
    __syncthreads();
    const int e = s_e[g];
    const int rg = lane >> 3, rl = lane & 7, q = rg >> 1;
    const int64_t j = hb * 32 + 4 * wave + q;
    const bool w3row = rg & 1;
    int4 c0[BU], c1[BU];
    float sw[BU];
    lane_row_load_pair<BU>(c0, c1, sw, static_cast<const uint8_t *>(stab[(w3row ? 2 : 0) * E + e]) + j * dim,
                      static_cast<const float *>(stab[(w3row ? 3 : 1) * E + e]) + j * nb, nb, rl);
    const float v = tree8_pair(lane_running_sum_pair<BU, EX>(c0, c1, sw, sq, sxs, nb, rl));
    const float v3 = row_shl8(v);  // lane 16q: the W3 dot of row q
    if (wave == 0) ffn1_wait_line(a, tag, kFfn1MaxK, nullptr, s_w);
    __syncthreads();
    if ((lane & 15) == 0) sh[4 * wave + q] = s_w[g] * silu_mul(v, v3);
    __syncthreads();
    if (wave == 0) {
        const float4 v4 = reinterpret_cast<const float4 *>(sh)[min(lane, 7)];
        float d;
        int cs;
        const uint32_t pk = quantize_group(v4.x, v4.y, v4.z, v4.w, d, cs);
        tag_put_q8(a.hw + 6 * ((int64_t)g * nhb + hb), pk, d, tag);
    }
}

// y_t = Σ o over the token's experts in ascending index, from +0; out_t = y_t,
// or Canonical(out_t + y_t) (the layer's residual, model.go:608-610).
__global__ __launch_bounds__(256) void moe_combine_kernel(const int32_t *sel, int k, const float *o, int dim,
                                                          float *out, int residual) {
    __shared__ int order[kMoeMaxK];  // the token's slots by ascending expert
    const int t = blockIdx.x;
    if ((int)threadIdx.x < k) {
        // a token's experts are distinct: slot s goes to place #{s': sel[s'] < sel[s]}
        const int32_t *ts = sel + (int64_t)t * k;
        const int e = ts[threadIdx.x];
        int r = 0;
        for (int q = 0; q < k; q++) r += ts[q] < e;
        order[r] = threadIdx.x;
    }
    __syncthreads();
    const int i = blockIdx.y * 256 + threadIdx.x;
    if (i >= dim) return;
    float acc = 0.0f;
    for (int s = 0; s < k; s++) acc += o[((int64_t)t * k + order[s]) * dim + i];
    float *dst = out + (int64_t)t * dim + i;
    *dst = residual ? canonical(*dst + acc) : acc;
}

// The ascending-order sum into the residual (moe_combine_kernel's steps),
// then RMSNorm of each new row with the next layer's weights and its Q8_0
// form (norm_quant_kernel's steps): one workgroup a token, four values a
// thread.
constexpr int kCnThreads = 1024;
constexpr int kCnGroups = (kMaxNormCols / 4 + kCnThreads - 1) / kCnThreads;
__global__ __launch_bounds__(kCnThreads) void moe_combine_norm_kernel(const int32_t *sel, int k, const float *o,
                                                                      int dim, float *out, const float *norm_w,
                                                                      float recip_n, float eps, int8_t *qx, float *xs,
                                                                      int32_t *xsum) {
    extern __shared__ __align__(16) float sxn[];
    __shared__ float bcast;
    __shared__ int order[kMoeMaxK];  // the token's slots by ascending expert
    const int t = blockIdx.x, tid = threadIdx.x;
    if (tid < k) {
        const int32_t *ts = sel + (int64_t)t * k;
        const int e = ts[tid];
        int r = 0;
        for (int q = 0; q < k; q++) r += ts[q] < e;
        order[r] = tid;
    }
    __syncthreads();
    const int ng = dim >> 2;
    float4 xv[kCnGroups], wv[kCnGroups];
#pragma unroll
    for (int kk = 0; kk < kCnGroups; kk++) {
        const int gu = tid + kk * kCnThreads, g = min(gu, ng - 1);
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int q = 0; q < k; q++) {
            const float4 ov = reinterpret_cast<const float4 *>(o + ((int64_t)t * k + order[q]) * dim)[g];
            acc.x += ov.x;
            acc.y += ov.y;
            acc.z += ov.z;
            acc.w += ov.w;
        }
        float4 *dst = reinterpret_cast<float4 *>(out + (int64_t)t * dim) + g;
        const float4 x0 = *dst;
        const float4 x1 = make_float4(canonical(x0.x + acc.x), canonical(x0.y + acc.y), canonical(x0.z + acc.z),
                                      canonical(x0.w + acc.w));
        if (gu < ng) *dst = x1;
        xv[kk] = x1;
        wv[kk] = reinterpret_cast<const float4 *>(norm_w)[g];
    }
    wg_norm_quant<kCnThreads, kCnGroups>(xv, wv, dim, recip_n, eps, qx + (int64_t)t * dim,
                                          xs + (int64_t)t * (dim >> 5), xsum + (int64_t)t * (dim >> 5), sxn, &bcast);
}

}  // namespace

int64_t moe_sync_words(const rk_moe *m) { return ffn1_sync_layout(m->dim, m->experts, m->topk, m->hidden).words; }

int64_t moe_scratch_layout(const rk_moe *m, int cap, char *mem, MoeScratch *sc) {
    const int64_t T = cap, K = m->topk, E = m->experts, D = m->dim, H = m->hidden;
    const int64_t G = std::min<int64_t>(E, T * K);
    int64_t at = 0;
    auto take = [&](int64_t bytes) {
        const int64_t here = at;
        at += (bytes + 255) & ~(int64_t)255;
        return mem ? mem + here : nullptr;
    };
    MoeScratch s;
    s.cap = cap;
    s.gcap = (int)G;
    s.logits = reinterpret_cast<float *>(take(4 * T * E));
    s.sel = reinterpret_cast<int32_t *>(take(4 * T * K));
    s.wsel = reinterpret_cast<float *>(take(4 * T * K));
    s.grp = reinterpret_cast<int32_t *>(take(4 * (1 + 3 * G + T * K)));
    s.gwt = reinterpret_cast<float *>(take(4 * T * K));
    s.gptr = reinterpret_cast<const void **>(take(8 * 6 * G));
    s.hq = reinterpret_cast<int8_t *>(take(T * K * H));
    s.hs = reinterpret_cast<float *>(take(4 * T * K * (H / 32)));
    s.hsum = reinterpret_cast<int32_t *>(take(4 * T * K * (H / 32)));
    s.o = reinterpret_cast<float *>(take(4 * T * K * D));
    if (sc) *sc = s;
    return at;
}

static int enqueue_moe_experts(rk_moe *m, const MoeScratch &sc, const int8_t *qx, const float *xs, int tokens,
                               float *out, bool residual, hipStream_t s, const MoeNext *next = nullptr);
static int enqueue_moe_down(rk_moe *m, const MoeScratch &sc, int tokens, float *out, bool residual, hipStream_t s,
                            const MoeNext *next = nullptr);

int enqueue_moe_q(rk_moe *m, const MoeScratch &sc, const int8_t *qx, const float *xs, const int32_t *xsum, int tokens,
                  float *out, bool residual, hipStream_t s, const MoeNext *next) {
    rk_device *d = m->d;
    const int D = m->dim, K = m->topk, E = m->experts;
    if (tokens <= 0) return RK_OK;
    if (tokens > sc.cap) return fail(d, RK_ERR_ARGS, "moe: %d tokens beyond the scratch's %d", tokens, sc.cap);
    bool ok;
    if (tokens == 1) {
        FusedArgs a{};
        a.seg[0] = MatSeg{m->router->w, m->router->scales, sc.logits, m->router->rows};
        a.nseg = 1;
        a.cols = D;
        a.rows = E;
        a.qx = qx;
        a.xs = xs;
        a.xsum = xsum;
        ProfScope p(d, s, "moe_router");
        ok = launch_fused(kFmtQ8, kProGlobal, kEpStore, a, d->cu, s);
    } else if (tokens <= kRouterMaxT && D <= 32 * 8 * kRouterBpl) {
        ProfScope p(d, s, "moe_router");
        RK_LAUNCH(moe_router_rows_kernel, dim3((unsigned)((E + 3) / 4)), dim3(256),
                  (size_t)tokens * D + (size_t)tokens * (D / 32) * 4, s, m->router->w, m->router->scales, E, D, qx,
                  xs, tokens, sc.logits);
        ok = true;
    } else {
        MmArgs a{};
        a.seg[0] = MatSeg{m->router->w, m->router->scales, sc.logits, m->router->rows};
        a.nseg = 1;
        a.cols = D;
        a.rows = E;
        a.tokens = tokens;
        a.qx = qx;
        a.xs = xs;
        ProfScope p(d, s, "moe_router");
        ok = launch_mm(kFmtQ8, kEpStore, a, s);
    }
    if (!ok) return fail(d, RK_ERR_UNSUPPORTED, "rk_moe: the router's product has no kernel");
    const int npairs = tokens * K;
    const MoeTabs tabs{m->w1, m->w3, m->w2, m->s1, m->s3, m->s2, sc.stat};
    if (tokens <= kSelectTokens && npairs <= kGroupFastPairs && E <= 1024) {
        static std::once_flag once;
        std::call_once(once, [] {
            (void)hipFuncSetAttribute((const void *)moe_select_kernel<kRoutePer>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kSelectTokens * 1024 * 4);
        });
        ProfScope p(d, s, "moe_select");
        const size_t lds = (size_t)tokens * ((E + 3) & ~3) * 4;
        if (E <= 128)
            RK_LAUNCH(moe_select_kernel<2>, dim3(1), dim3(1024), lds, s, sc.logits, tokens, E, K, sc.sel, sc.wsel,
                      sc.gcap, sc.grp, sc.gwt, tabs, sc.gptr);
        else
            RK_LAUNCH(moe_select_kernel<kRoutePer>, dim3(1), dim3(1024), lds, s, sc.logits, tokens, E, K, sc.sel,
                      sc.wsel, sc.gcap, sc.grp, sc.gwt, tabs, sc.gptr);
        return enqueue_moe_experts(m, sc, qx, xs, tokens, out, residual, s, next);
    }
    {
        ProfScope p(d, s, "moe_route");
        const size_t lds = (size_t)((E + 3) & ~3) * 4;
        if (E <= 128)
            RK_LAUNCH(moe_route_kernel<2>, dim3(tokens), dim3(64), lds, s, sc.logits, E, K, sc.sel, sc.wsel);
        else
            RK_LAUNCH(moe_route_kernel<kRoutePer>, dim3(tokens), dim3(64), lds, s, sc.logits, E, K, sc.sel, sc.wsel);
    }
    {
        ProfScope p(d, s, "moe_group");
        if (npairs <= kGroupFastPairs && E <= 1024)
            RK_LAUNCH(moe_group_fast_kernel, dim3(1), dim3(1024), 0, s, sc.sel, sc.wsel, npairs, E, sc.gcap, sc.grp,
                      sc.gwt, tabs, sc.gptr);
        else
            RK_LAUNCH(moe_group_kernel, dim3(1), dim3(1024), 0, s,
                      sc.sel, sc.wsel, npairs, E, sc.gcap, sc.grp, sc.gwt, tabs, sc.gptr);
    }
    return enqueue_moe_experts(m, sc, qx, xs, tokens, out, residual, s, next);
}

// The experts' products and sum after the routing (grouping in sc.grp).
static int enqueue_moe_experts(rk_moe *m, const MoeScratch &sc, const int8_t *qx, const float *xs, int tokens,
                               float *out, bool residual, hipStream_t s, const MoeNext *next) {
    rk_device *d = m->d;
    const int D = m->dim, H = m->hidden, K = m->topk, E = m->experts;
    const int groups = std::min(E, tokens * K);  // launched; those past the selected count exit
    {
        ProfScope p(d, s, "moe_up");
        const int bpl = (D / 32 + 7) / 8;  // blocks of a W1/W3 row per lane
        const dim3 grid8((unsigned)(H / 32), (unsigned)groups), grid((unsigned)groups, (unsigned)(H / 32));
        const bool all = tokens <= kExpTok;
        const size_t lds = (size_t)up8_lds(D);
        const bool ex = D / 32 == 8 * (bpl <= 2 ? 2 : bpl <= 4 ? 4 : 8);  // rows of exactly 8·B blocks
#define RK_UP8(B, A)                                                                                                    \
    do {                                                                                                                \
        if (ex)                                                                                                         \
            RK_LAUNCH((moe_up8_kernel<B, A, true>), grid8, dim3(512), lds, s, sc.gptr, sc.grp, sc.gcap, sc.gwt, K, qx,  \
                      xs, tokens, D, H, sc.hq, sc.hs, sc.hsum);                                                         \
        else                                                                                                            \
            RK_LAUNCH((moe_up8_kernel<B, A, false>), grid8, dim3(512), lds, s, sc.gptr, sc.grp, sc.gcap, sc.gwt, K, qx, \
                      xs, tokens, D, H, sc.hq, sc.hs, sc.hsum);                                                         \
    } while (0)
        if (bpl <= 2) {
            if (all) RK_UP8(2, true);
            else RK_UP8(2, false);
        } else if (bpl <= 4) {
            if (all) RK_UP8(4, true);
            else RK_UP8(4, false);
        } else if (bpl <= 8) {
            if (all) RK_UP8(8, true);
            else RK_UP8(8, false);
        } else {
            RK_LAUNCH(moe_up_kernel, grid, dim3(512), 0, s, m->w1, m->s1, m->w3, m->s3, sc.grp, sc.gcap, sc.wsel, K, qx,
                      xs, D, H, sc.hq, sc.hs, sc.hsum);
        }
#undef RK_UP8
    }
    return enqueue_moe_down(m, sc, tokens, out, residual, s, next);
}

// The W2 products of the grouped pairs (h in sc) and the sum (with `next`:
// and the next product's input).
static int enqueue_moe_down(rk_moe *m, const MoeScratch &sc, int tokens, float *out, bool residual, hipStream_t s,
                            const MoeNext *next) {
    rk_device *d = m->d;
    const int D = m->dim, H = m->hidden, K = m->topk, E = m->experts;
    const int groups = std::min(E, tokens * K);  // launched; those past the selected count exit
    {
        ProfScope p(d, s, "moe_down");
        const int bpl = (H / 32 + 7) / 8;  // blocks of a W2 row per lane
        const size_t lds = (size_t)kExpTok * (H + (H / 32) * 4 + 4);
        const dim3 grid((unsigned)((D + 31) / 32), (unsigned)groups);
#define RK_DOWN8(B, X)                                                                                       \
    RK_LAUNCH((moe_down8_kernel<B, X>), grid, dim3(256), lds, s, sc.gptr, sc.grp, sc.gcap, sc.hq, sc.hs, D, H, sc.o)
        const int nbh = H / 32;  // rows of exactly 8·B blocks take the unclamped form
        if (bpl <= 2) {
            if (nbh == 16) RK_DOWN8(2, true);
            else RK_DOWN8(2, false);
        } else if (bpl <= 3 && nbh == 24) {
            RK_DOWN8(3, true);
        } else if (bpl <= 4) {
            if (nbh == 32) RK_DOWN8(4, true);
            else RK_DOWN8(4, false);
        } else if (bpl <= 8) {
            if (nbh == 64) RK_DOWN8(8, true);
            else RK_DOWN8(8, false);
        } else {
            RK_LAUNCH(moe_down_kernel, dim3((unsigned)groups, (unsigned)((D + 15) / 16)), dim3(256), 0, s, m->w2,
                      m->s2, sc.grp, sc.gcap, sc.hq, sc.hs, D, H, sc.o);
        }
#undef RK_DOWN8
    }
    if (next && residual && D % 32 == 0 && D <= kMaxNormCols) {
        ProfScope p(d, s, "moe_combine");
        RK_LAUNCH(moe_combine_norm_kernel, dim3((unsigned)tokens), dim3(kCnThreads), norm_lds(D), s, sc.sel, K, sc.o,
                  D, out, next->norm_w, next->recip_n, next->eps, next->qx, next->xs, next->xsum);
    } else {
        ProfScope p(d, s, "moe_combine");
        RK_LAUNCH(moe_combine_kernel, dim3((unsigned)tokens, (unsigned)((D + 255) / 256)), dim3(256), 0, s, sc.sel, K,
                  sc.o, D, out, residual ? 1 : 0);
        if (next) {
            ProfScope p2(d, s, "norm_quant");
            launch_norm_quant(out, D, next->norm_w, next->recip_n, next->eps, next->qx, next->xs, next->xsum, s,
                              tokens);
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(d, e, "moe launch");
    return RK_OK;
}

int enqueue_moe_x(rk_moe *m, const MoeScratch &sc, const float *x, const float *norm_w, float recip_n, float eps,
                  int tokens, int8_t *qx, float *xs, int32_t *xsum, float *out, bool residual, hipStream_t s,
                  const MoeNext *next) {
    rk_device *d = m->d;
    if (tokens <= 0) return RK_OK;
    if (tokens > sc.cap) return fail(d, RK_ERR_ARGS, "moe: %d tokens beyond the scratch's %d", tokens, sc.cap);
    const int D = m->dim, E = m->experts, K = m->topk, H = m->hidden;
    if (norm_w && tokens == 1 && !next && sc.sync && sc.err && D <= kFfn1MaxCols && E <= kFfn1MaxExperts &&
        K <= kFfn1MaxK && H <= kFfn1MaxHidden) {
        // one token, the whole feed-forward in one launch
        Ffn1Args a{};
        a.x = x;
        a.norm_w = norm_w;
        a.recip_n = recip_n;
        a.eps = eps;
        a.rw = m->router->w;
        a.rws = m->router->scales;
        a.w1 = m->w1;
        a.w3 = m->w3;
        a.w2 = m->w2;
        a.s1 = m->s1;
        a.s3 = m->s3;
        a.s2 = m->s2;
        a.experts = E;
        a.k = K;
        a.dim = D;
        a.hidden = H;
        const Ffn1Sync sy = ffn1_sync_layout(D, E, K, H);
        a.lines = sc.sync + sy.lines;
        a.lw = sc.sync + sy.lw;
        a.hw = sc.sync + sy.hw;
        a.cnt = sc.sync + sy.cnt;
        a.sel = sc.sel;
        a.wsel = sc.wsel;
        a.out = out;
        a.residual = residual ? 1 : 0;
        a.err = sc.err;
        a.nr = (E + 7) / 8;
        a.nu = K * (H / 32);
        a.nd = (D + 64 / K - 1) / (64 / K);
        const size_t lds = (size_t)ffn1_lds(D, E, K, H).bytes;
        const int bu = (D / 32 + 7) / 8, bd = (H / 32 + 7) / 8;
        const dim3 grid((unsigned)(a.nr + a.nu + a.nd));
        typedef void (*Ffn1Fn)(Ffn1Args);
#define RK_FFN1_ROW(U, X)                                                                                    \
    {moe_ffn1_kernel<U, 2, X>, moe_ffn1_kernel<U, 3, X>, moe_ffn1_kernel<U, 4, X>, moe_ffn1_kernel<U, 8, X>}
        static const Ffn1Fn fns[2][3][4] = {{RK_FFN1_ROW(2, false), RK_FFN1_ROW(4, false), RK_FFN1_ROW(8, false)},
                                            {RK_FFN1_ROW(2, true), RK_FFN1_ROW(4, true), RK_FFN1_ROW(8, true)}};
#undef RK_FFN1_ROW
        const int iu = bu <= 2 ? 0 : bu <= 4 ? 1 : 2, id = bd <= 2 ? 0 : bd <= 3 ? 1 : bd <= 4 ? 2 : 3;
        const int BUs[3] = {2, 4, 8}, BDs[4] = {2, 3, 4, 8};
        const bool ex = D / 32 == 8 * BUs[iu] && H / 32 == 8 * BDs[id];  // rows of exactly 8·B blocks
        const Ffn1Fn fn = fns[ex ? 1 : 0][iu][id];
        if (lds > 64 * 1024) {
            hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return hip_fail(d, e, "moe launch");
        }
        ProfScope p(d, s, "moe_ffn");
        RK_LAUNCH(fn, grid, dim3(512), lds, s, a);
        hipError_t e = hipGetLastError();
        return e == hipSuccess ? RK_OK : hip_fail(d, e, "moe launch");
    }
    if (norm_w && tokens == 1 && D <= 2048 && E <= kUp1MaxExperts && K <= kMoeMaxK) {
        // one token: the router's product with the RMSNorm in its prologue,
        // then the W1/W3 rows with the routing and the norm folded in (the
        // normed input is never stored: qx, xs and xsum are left as they are)
        FusedArgs a{};
        a.seg[0] = MatSeg{m->router->w, m->router->scales, sc.logits, m->router->rows};
        a.nseg = 1;
        a.cols = D;
        a.rows = E;
        a.x = x;
        a.norm_w = norm_w;
        a.recip_n = recip_n;
        a.norm_eps = eps;
        bool ok;
        {
            ProfScope p(d, s, "moe_router");
            ok = launch_fused(kFmtQ8, kProNorm, kEpStore, a, d->cu, s);
        }
        if (!ok) return fail(d, RK_ERR_UNSUPPORTED, "rk_moe: the router's product has no kernel");
        const int bpl = (D / 32 + 7) / 8;
        const size_t lds = (size_t)up1_lds(D, E).bytes;
        {
            ProfScope p(d, s, "moe_up");
#define RK_UP1(B)                                                                                                  \
    RK_LAUNCH((moe_up1_kernel<B>), dim3((unsigned)K, (unsigned)(H / 32)), dim3(512), lds, s, x, norm_w, recip_n,     \
              eps, sc.logits, E, K, m->w1, m->s1, m->w3, m->s3, m->w2, m->s2, D, H, sc.sel, sc.wsel, sc.gcap,       \
              sc.grp, sc.gptr, sc.hq, sc.hs, sc.hsum)
            if (bpl <= 2) RK_UP1(2);
            else if (bpl <= 4) RK_UP1(4);
            else RK_UP1(8);
#undef RK_UP1
        }
        if (H / 32 > 8 * 8) return enqueue_moe_down(m, sc, tokens, out, residual, s, next);
        {
            ProfScope p(d, s, "moe_down");
            const int R = 64 / K, hbpl = (H / 32 + 7) / 8;
            const dim3 grid((unsigned)((D + R - 1) / R));
            if (hbpl <= 2)
                RK_LAUNCH(moe_down1_kernel<2>, grid, dim3(512), 0, s, sc.gptr, sc.grp, sc.gcap, K, sc.hq, sc.hs, D,
                          H, out, residual ? 1 : 0);
            else if (hbpl <= 4)
                RK_LAUNCH(moe_down1_kernel<4>, grid, dim3(512), 0, s, sc.gptr, sc.grp, sc.gcap, K, sc.hq, sc.hs, D,
                          H, out, residual ? 1 : 0);
            else
                RK_LAUNCH(moe_down1_kernel<8>, grid, dim3(512), 0, s, sc.gptr, sc.grp, sc.gcap, K, sc.hq, sc.hs, D,
                          H, out, residual ? 1 : 0);
        }
        if (next) {
            ProfScope p(d, s, "norm_quant");
            launch_norm_quant(out, D, next->norm_w, next->recip_n, next->eps, next->qx, next->xs, next->xsum, s, 1);
        }
        hipError_t e = hipGetLastError();
        return e == hipSuccess ? RK_OK : hip_fail(d, e, "moe launch");
    }
    if (norm_w) {
        ProfScope p(d, s, "norm_quant");
        launch_norm_quant(x, m->dim, norm_w, recip_n, eps, qx, xs, xsum, s, tokens);
    } else {
        ProfScope p(d, s, "quantize_acts");
        launch_quantize_acts(x, (int64_t)tokens * m->dim, qx, xs, xsum, s);
    }
    return enqueue_moe_q(m, sc, qx, xs, xsum, tokens, out, residual, s, next);
}

// The standalone calls' scratch for up to `tokens` inputs (grown: a call
// that must grow it cannot be recorded).
static int moe_own_scratch(rk_moe *m, int tokens) {
    if (tokens <= m->cap) return RK_OK;
    rk_device *d = m->d;
    if (d->capturing) return fail(d, RK_ERR_ARGS, "rk_moe: scratch must grow, which cannot be recorded");
    HIP_TRY(d, hipDeviceSynchronize(), "moe scratch");
    (void)hipFree(m->mem);
    m->mem = nullptr;
    add_used(d, -m->bytes);
    m->bytes = 0;
    m->cap = 0;
    const int64_t T = std::max(tokens, 16), D = m->dim;
    auto al = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
    const int64_t own = 2 * al(4 * T * D) + al(T * D) + 2 * al(4 * T * (D / 32));
    const int64_t total = own + moe_scratch_layout(m, (int)T, nullptr, nullptr);
    int rc = dev_alloc(d, &m->mem, (size_t)total, "moe scratch");
    if (rc) return rc;
    char *p = static_cast<char *>(m->mem);
    m->x = reinterpret_cast<float *>(p);
    p += al(4 * T * D);
    m->y = reinterpret_cast<float *>(p);
    p += al(4 * T * D);
    m->qx = reinterpret_cast<int8_t *>(p);
    p += al(T * D);
    m->xs = reinterpret_cast<float *>(p);
    p += al(4 * T * (D / 32));
    m->xsum = reinterpret_cast<int32_t *>(p);
    p += al(4 * T * (D / 32));
    moe_scratch_layout(m, (int)T, p, &m->sc);
    m->bytes = total;
    m->cap = (int)T;
    add_used(d, m->bytes);
    return RK_OK;
}

// A standalone call: the input quantized into the handle's scratch, then
// the feed-forward into d_y.
static int enqueue_moe(rk_moe *m, const float *d_xn, int tokens, float *d_y, hipStream_t s) {
    return enqueue_moe_x(m, m->sc, d_xn, nullptr, 0.0f, 0.0f, tokens, m->qx, m->xs, m->xsum, d_y, false, s);
}

}  // namespace rk

using namespace rk;

extern "C" {

int rk_moe_new(rk_device *d, rk_matrix *router, int32_t experts, rk_matrix *const *w1, rk_matrix *const *w2,
               rk_matrix *const *w3, int32_t topk, rk_moe **out) {
    if (!d || !out || !router || !w1 || !w2 || !w3) return fail(d, RK_ERR_ARGS, "rk_moe_new: null argument");
    *out = nullptr;
    if (experts <= 0 || experts > kMoeMaxExperts || topk <= 0 || topk > kMoeMaxK || topk > experts)
        return fail(d, RK_ERR_ARGS, "rk_moe_new: %d experts, top %d", experts, topk);
    const int64_t dim = router->cols, hidden = w1[0] ? w1[0]->rows : 0;
    if (router->d != d || router->rows != experts || router->kind != RK_Q8)
        return fail(d, RK_ERR_ARGS, "rk_moe_new: the router must be a Q8 %d-row matrix on the device", experts);
    if (dim > kMoeMaxCols || hidden <= 0 || hidden > kMoeMaxCols || dim % 32 || hidden % 32)
        return fail(d, RK_ERR_UNSUPPORTED, "rk_moe_new: dim %lld / hidden %lld", (long long)dim, (long long)hidden);
    for (int e = 0; e < experts; e++) {
        const rk_matrix *a = w1[e], *b = w3[e], *c = w2[e];
        if (!a || !b || !c || a->d != d || b->d != d || c->d != d || a->kind != RK_Q8 || b->kind != RK_Q8 ||
            c->kind != RK_Q8 || a->rows != hidden || a->cols != dim || b->rows != hidden || b->cols != dim ||
            c->rows != dim || c->cols != hidden)
            return fail(d, RK_ERR_ARGS, "rk_moe_new: expert %d: W1/W3 %lldx%lld and W2 %lldx%lld Q8 matrices expected",
                        e, (long long)hidden, (long long)dim, (long long)dim, (long long)hidden);
    }
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    rk_moe *m = new rk_moe();
    m->d = d;
    m->router = router;
    m->experts = experts;
    m->topk = topk;
    m->dim = (int32_t)dim;
    m->hidden = (int32_t)hidden;
    std::vector<const void *> tab(6 * (size_t)experts);
    for (int e = 0; e < experts; e++) {
        tab[e] = w1[e]->w;
        tab[experts + e] = w3[e]->w;
        tab[2 * experts + e] = w2[e]->w;
        tab[3 * experts + e] = w1[e]->scales;
        tab[4 * experts + e] = w3[e]->scales;
        tab[5 * experts + e] = w2[e]->scales;
    }
    int rc = dev_alloc(d, &m->tables, tab.size() * sizeof(void *), "moe tables");
    if (rc) {
        delete m;
        return rc;
    }
    const void **t = static_cast<const void **>(m->tables);
    m->w1 = reinterpret_cast<const uint8_t **>(t);
    m->w3 = reinterpret_cast<const uint8_t **>(t + experts);
    m->w2 = reinterpret_cast<const uint8_t **>(t + 2 * experts);
    m->s1 = reinterpret_cast<const float **>(t + 3 * experts);
    m->s3 = reinterpret_cast<const float **>(t + 4 * experts);
    m->s2 = reinterpret_cast<const float **>(t + 5 * experts);
    hipError_t e = hipMemcpy(m->tables, tab.data(), tab.size() * sizeof(void *), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(m->tables);
        delete m;
        return hip_fail(d, e, "moe tables");
    }
    *out = m;
    return RK_OK;
}

int rk_moe_ffn(rk_moe *m, const float *xn, int32_t tokens, float *y, int32_t *sel, float *wsel) {
    if (!m) return RK_ERR_ARGS;
    rk_device *d = m->d;
    if (tokens < 0 || (tokens > 0 && (!xn || !y))) return fail(d, RK_ERR_ARGS, "rk_moe_ffn: bad arguments");
    if (tokens == 0) return RK_OK;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    if (d->capturing) return fail(d, RK_ERR_ARGS, "rk_moe_ffn waits for its results: it cannot be recorded");
    int rc = moe_own_scratch(m, tokens);
    if (rc) return rc;
    hipStream_t s = d->stream;
    const size_t xb = (size_t)tokens * m->dim * 4;
    HIP_TRY(d, hipMemcpyAsync(m->x, xn, xb, hipMemcpyHostToDevice, s), "moe input");
    if ((rc = enqueue_moe(m, m->x, tokens, m->y, s))) return rc;
    HIP_TRY(d, hipMemcpyAsync(y, m->y, xb, hipMemcpyDeviceToHost, s), "moe output");
    if (sel)
        HIP_TRY(d, hipMemcpyAsync(sel, m->sc.sel, (size_t)tokens * m->topk * 4, hipMemcpyDeviceToHost, s), "moe sel");
    if (wsel)
        HIP_TRY(d, hipMemcpyAsync(wsel, m->sc.wsel, (size_t)tokens * m->topk * 4, hipMemcpyDeviceToHost, s), "moe w");
    HIP_TRY(d, hipStreamSynchronize(s), "moe");
    return RK_OK;
}

int rk_moe_ffn_device(rk_moe *m, const float *d_xn, int32_t tokens, float *d_y, void *stream) {
    if (!m) return RK_ERR_ARGS;
    rk_device *d = m->d;
    if (tokens < 0 || (tokens > 0 && (!d_xn || !d_y))) return fail(d, RK_ERR_ARGS, "rk_moe_ffn_device: bad arguments");
    if (tokens == 0) return RK_OK;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    hipStream_t s = stream ? (hipStream_t)stream : d->stream;
    if (d->capturing && s != d->stream)
        return fail(d, RK_ERR_ARGS, "while recording a graph, work goes on the device's stream");
    int rc = moe_own_scratch(m, tokens);
    if (rc) return rc;
    return enqueue_moe(m, d_xn, tokens, d_y, s);
}

int64_t rk_moe_bytes(const rk_moe *m) { return m ? m->bytes : -1; }

int rk_moe_free(rk_moe *m) {
    if (!m) return RK_ERR_ARGS;
    rk_device *d = m->d;
    Hold hold(d->gate);
    (void)hipSetDevice(d->index);
    (void)hipStreamSynchronize(d->stream);
    (void)hipFree(m->tables);
    (void)hipFree(m->mem);
    add_used(d, -m->bytes);
    delete m;
    return RK_OK;
}

}  // extern "C"
