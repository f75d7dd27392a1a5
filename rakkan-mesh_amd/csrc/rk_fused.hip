// rk_fused.hip — fused quantized products and the attention of one position,
// for gfx950. Results are the CPU path's bits (internal/num, internal/llm):
//
// Product (internal/num/quant.go:14-19, 158-196): the input is quantized to
// Q8_0; block b of a row contributes float32(sum_b)·float32(ws_b·xs_b) to
// running sum b mod 8, in order of b, and the eight sums combine as
// ((0+1)+(2+3))+((4+5)+(6+7)). sum_b is an exact integer (v_dot4), so only
// the float steps are ordered.
//
// Work layout: a workgroup owns a contiguous run of output rows; its waves
// take rows (or adjacent row pairs, when the epilogue needs both) in turn.
// A wave streams a row in 1 KiB chunks of codes, one 16-byte piece per lane
// (coalesced global_load_dwordx4), keeping U chunks in flight. The input's
// quantized form is either read like the weights (kProGlobal) or made by
// the workgroup itself into LDS before the stream starts (kProQuant): the
// input's loads are issued first, then the first weight chunks, so the
// prologue runs while those weights are on their way. Results wait in LDS
// and leave coalesced at the end.
#include <algorithm>
#include <mutex>

#include "rk_dev.h"
#include "rk_fused.h"
#include "rk_sync.h"

namespace rk {

namespace {

struct RowSrc {
    const uint8_t *w;
    const float *ws;
    float *out;
    int r;
};

// Source of logical row l: three concatenated matrices, or (kEpSilu) two
// interleaved row by row. Uniform selects keep the table in SGPRs.
template <int EPI>
__device__ __forceinline__ RowSrc row_src(const FusedArgs &a, int l, int rowbytes, int nb) {
    RowSrc s;
    if (EPI == kEpSilu) {
        const bool odd = l & 1;
        s.r = l >> 1;
        s.w = odd ? a.seg[1].w : a.seg[0].w;
        s.ws = odd ? a.seg[1].ws : a.seg[0].ws;
        s.out = nullptr;
    } else {
        s.r = l;
        s.w = a.seg[0].w;
        s.ws = a.seg[0].ws;
        s.out = a.seg[0].out;
        if (a.nseg > 1 && s.r >= a.seg[0].rows) {
            s.r -= a.seg[0].rows;
            s.w = a.seg[1].w;
            s.ws = a.seg[1].ws;
            s.out = a.seg[1].out;
            if (a.nseg > 2 && s.r >= a.seg[1].rows) {
                s.r -= a.seg[1].rows;
                s.w = a.seg[2].w;
                s.ws = a.seg[2].ws;
                s.out = a.seg[2].out;
            }
        }
    }
    s.w += (int64_t)s.r * rowbytes;
    s.ws += (int64_t)s.r * nb;
    return s;
}

}  // namespace

template <int FMT, int PRO, int EPI, int W, int U>
__global__ __launch_bounds__(64 * W) void fused_kernel(FusedArgs a) {
    extern __shared__ __align__(16) char lds[];
    __shared__ float s_wv[W];
    __shared__ int s_wi[W];
    constexpr bool PAIR = (EPI == kEpQKV || EPI == kEpSilu);
    // epilogues that need one value per row read before the stream: the
    // output being added to, or the row's bias
    constexpr bool PRE = (EPI == kEpAdd || EPI == kEpAddCanon || EPI == kEpStore || EPI == kEpQKV);
    constexpr int NT = 64 * W;
    constexpr int MAXG = PRO == kProGlobal ? 1
                         : PRO == kProNorm ? (kMaxNormProCols / 4 + NT - 1) / NT
                                           : (kMaxLdsCols / 4 + NT - 1) / NT;
    __shared__ float s_rn;  // kProNorm: the broadcast Rsqrt32
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cols = a.cols, nb = cols >> 5;
    const int rowbytes = FMT == kFmtQ8 ? cols : cols >> 1;
    const int C = FMT == kFmtQ8 ? (cols + 1023) >> 10 : (nb + 63) >> 6;

    int pos = 0;
    if (EPI == kEpQKV || EPI == kEpLogits) pos = a.ctl[kCtlPos];
    const bool work = !(EPI == kEpLogits && a.gate && pos + 1 < a.ctl[kCtlPrompt]);

    const int R0 = blockIdx.x * a.rows_per_wg;
    const int R1 = min(a.rows, R0 + a.rows_per_wg);
    const int n = R1 - R0;  // >= 1: the launcher sizes the grid to the rows
    const int half = a.hs >> 1;
    int8_t *sqx = reinterpret_cast<int8_t *>(lds);
    float *sxs = reinterpret_cast<float *>(lds + a.lds_xs);
    int *sxsum = reinterpret_cast<int *>(lds + a.lds_xsum);
    float *sres = reinterpret_cast<float *>(lds + a.lds_res);  // the workgroup's results
    float *sep = reinterpret_cast<float *>(lds + a.lds_ep);    // per-row operands, then cos, sin
    float best_v = 0.0f;
    int best_i = -1;

    // Everything below keeps the main loop free of loads other than the
    // weight stream and of global stores, so each wait there is for the
    // oldest chunk only: the loads before it are unconditional (addresses
    // clamped into the buffers, unused values masked), per-row operands are
    // staged in LDS first and results leave through LDS at the end.
    if (work) {
        int nrows = 0;
        if (PAIR) {
            const int np = (n + 1) >> 1;
            if (wave < np) {
                nrows = 2 * ((np - 1 - wave) / W + 1);
                if ((n & 1) && (np - 1 - wave) % W == 0) nrows -= 1;
            }
        } else {
            nrows = wave < n ? (n - 1 - wave) / W + 1 : 0;
        }
        const int nsteps = nrows * C;
        // Row cursors: PAIR waves take pairs wave, wave+W, ... (both rows of
        // each, in order); the others rows wave, wave+W, ...
        auto row_of = [&](int p, int h) { return PAIR ? R0 + 2 * p + h : R0 + p; };
        auto next_row = [&](int &p, int &h) {
            if (PAIR) {
                if (h == 0 && R0 + 2 * p + 1 < R1) {
                    h = 1;
                } else {
                    p += W;
                    h = 0;
                }
            } else {
                p += W;
            }
        };

        // ---- (1) loads the prologue needs: the input (and norm weights),
        // the rows' epilogue operands, the rotary row ----
        float4 xv[MAXG], wv[MAXG];
        if (PRO != kProGlobal) {
            const int ng = cols >> 2;
#pragma unroll
            for (int k = 0; k < MAXG; k++) {
                const int g = min((int)threadIdx.x + k * NT, ng - 1);
                xv[k] = reinterpret_cast<const float4 *>(a.x)[g];
                if (PRO == kProNorm) wv[k] = reinterpret_cast<const float4 *>(a.norm_w)[g];
            }
        }
        float epv = 0.0f, cosv = 0.0f, sinv = 0.0f;
        if (PRE) {
            const int i = min((int)threadIdx.x, n - 1);
            const bool add = EPI == kEpAdd || EPI == kEpAddCanon;
            // no bias: read a word known to exist, unused
            const float *src = add ? a.seg[0].out + R0 : a.bias ? a.bias + a.row_base + R0 : a.seg[0].ws;
            epv = src[(add || a.bias) ? i : 0];
            if (EPI == kEpQKV) {
                const int p = min((int)threadIdx.x, half - 1);
                cosv = a.cos_t[(int64_t)pos * half + p];
                sinv = a.sin_t[(int64_t)pos * half + p];
            }
        }

        // ---- (2) the weight stream: U chunks in flight ----
        int lp = wave, lh = 0, lc = 0, lstep = 0;
        RowSrc ls = row_src<EPI>(a, nsteps > 0 ? row_of(lp, lh) : 0, rowbytes, nb);
        int4 wb[U], xb0[U], xb1[U];
        float sb[U], xsb[U];
        int xsumb[U];
        // Lanes past a row's end read a clamped address: their blocks are
        // excluded where terms are summed (b < nb), so their values need no
        // masking. A load past the wave's last step (the loop keeps U in
        // flight) reads the first words of the scales instead, which stay in
        // the caches; its values are never used.
        const uint8_t *dummy = reinterpret_cast<const uint8_t *>(a.seg[0].ws);
        auto load = [&](int j) {
            const bool live = lstep < nsteps;
            if (FMT == kFmtQ8) {
                const int o = min(lc * 1024 + lane * 16, cols - 16);
                const uint8_t *wp = live ? ls.w + o : dummy;
                const float *sp = live ? ls.ws + (o >> 5) : a.seg[0].ws;
                wb[j] = load_stream16(wp);
                sb[j] = *sp;
                if (PRO == kProGlobal) {
                    xb0[j] = *reinterpret_cast<const int4 *>(a.qx + o);
                    xsb[j] = a.xs[o >> 5];
                }
            } else {
                const int bk = min(lc * 64 + lane, nb - 1);
                const uint8_t *wp = live ? ls.w + bk * 16 : dummy;
                const float *sp = live ? ls.ws + bk : a.seg[0].ws;
                wb[j] = load_stream16(wp);
                sb[j] = *sp;
                if (PRO == kProGlobal) {
                    xb0[j] = *reinterpret_cast<const int4 *>(a.qx + bk * 32);
                    xb1[j] = *reinterpret_cast<const int4 *>(a.qx + bk * 32 + 16);
                    xsb[j] = a.xs[bk];
                    xsumb[j] = a.xsum[bk];
                }
            }
            ++lstep;
            if (++lc == C) {
                lc = 0;
                if (lstep < nsteps) {
                    next_row(lp, lh);
                    ls = row_src<EPI>(a, row_of(lp, lh), rowbytes, nb);
                }
            }
        };
#pragma unroll
        for (int j = 0; j < U; j++) load(j);

        // ---- (3) prologue: stage the operands; Q8_0 quantization
        // (internal/num/quant.go:34-53) of the input into LDS ----
        // the per-row operands matter only when added (a residual, a bias)
        const bool use_sep = PRE && (EPI == kEpAdd || EPI == kEpAddCanon || EPI == kEpQKV || a.bias != nullptr);
        if (use_sep) {
            if ((int)threadIdx.x < n) sep[threadIdx.x] = epv;
            if (EPI == kEpQKV && (int)threadIdx.x < half) {
                sep[a.rows_per_wg + threadIdx.x] = cosv;
                sep[a.rows_per_wg + half + threadIdx.x] = sinv;
            }
        }
        if (PRO == kProNorm) {
            // RMSNorm (Dot32 over x held transposed, Rsqrt32) and the Q8 of
            // w·(r·x), as the stand-alone norm kernel computes it
            wg_norm_quant<NT, MAXG>(xv, wv, cols, a.recip_n, a.norm_eps, sqx, sxs, sxsum,
                                    reinterpret_cast<float *>(lds + a.lds_norm), &s_rn);
        } else if (PRO == kProQuant) {
#pragma unroll
            for (int k = 0; k < MAXG; k++) {
                const int g = threadIdx.x + k * NT;
                if (k * NT < (cols >> 2)) {  // uniform: the group row holds some of x
                    float d;
                    int cs;
                    const uint32_t pk = quantize_group(xv[k].x, xv[k].y, xv[k].z, xv[k].w, d, cs);
                    if (g < (cols >> 2)) {
                        reinterpret_cast<uint32_t *>(sqx)[g] = pk;
                        if ((g & 7) == 0) {
                            sxs[g >> 3] = d;
                            sxsum[g >> 3] = cs;
                        }
                    }
                }
            }
        }
        if (use_sep || PRO != kProGlobal) __syncthreads();

        // ---- (4) stream, reduce, epilogue into LDS ----
        float acc = 0.0f, held = 0.0f;
        int pp = wave, ph = 0, pc = 0;
        const bool has_bias = a.bias != nullptr;
        auto epilogue = [&](int l, float res) {
            const int i = l - R0;
            if (EPI == kEpSilu) {
                if ((i & 1) == 0)
                    held = res;
                else
                    sres[i >> 1] = silu_mul(held, res);
            } else if (EPI == kEpQKV) {
                const float v = has_bias ? res + sep[i] : res;
                if ((i & 1) == 0) {
                    held = v;
                } else {
                    const float v0 = held, v1 = v;
                    const int i0 = a.row_base + l - 1;
                    if (i0 < a.qdim + a.kvdim) {
                        const int ih = i0 < a.qdim ? i0 : i0 - a.qdim;
                        const int pi = (ih % a.hs) >> 1;
                        const float co = sep[a.rows_per_wg + pi], si = sep[a.rows_per_wg + half + pi];
                        sres[i - 1] = (v0 * co) - (v1 * si);
                        sres[i] = (v0 * si) + (v1 * co);
                    } else {
                        sres[i - 1] = v0;
                        sres[i] = v1;
                    }
                }
            } else if (EPI == kEpStore) {
                sres[i] = has_bias ? res + sep[i] : res;
            } else if (EPI == kEpAdd) {
                sres[i] = sep[i] + res;
            } else if (EPI == kEpAddCanon) {
                sres[i] = canonical(sep[i] + res);
            } else if (EPI == kEpLogits) {
                sres[i] = res;
                if (res == res) argmax_merge(best_v, best_i, res, l);
            }
        };

        auto process = [&](int j) {
            float t;
            if (FMT == kFmtQ8) {
                int4 xq = xb0[j];
                float xsv = xsb[j];
                if (PRO != kProGlobal) {
                    const int off = min(pc * 1024 + lane * 16, cols - 16);
                    xq = *reinterpret_cast<const int4 *>(sqx + off);
                    xsv = sxs[off >> 5];
                }
                const int s = pair_sum(dot16(wb[j], xq, 0));
                t = (float)s * (sb[j] * xsv);
                // block 32pc+k is in lanes 2k, 2k+1; running sum L in lane 2L
                // takes blocks 32pc+L, +8, +16, +24 (lanes 2L, +16, +32, +48).
                const float t1 = __shfl_down(t, 16);
                const float t2 = __shfl_down(t, 32);
                const float t3 = __shfl_down(t, 48);
                if (lane < 16 && (lane & 1) == 0) {
                    const int b0 = pc * 32 + (lane >> 1);
                    if (b0 < nb) acc += t;
                    if (b0 + 8 < nb) acc += t1;
                    if (b0 + 16 < nb) acc += t2;
                    if (b0 + 24 < nb) acc += t3;
                }
            } else {
                int4 x0 = xb0[j], x1 = xb1[j];
                float xsv = xsb[j];
                int xsum = xsumb[j];
                if (PRO != kProGlobal) {
                    const int blk = min(pc * 64 + lane, nb - 1);
                    x0 = *reinterpret_cast<const int4 *>(sqx + blk * 32);
                    x1 = *reinterpret_cast<const int4 *>(sqx + blk * 32 + 16);
                    xsv = sxs[blk];
                    xsum = sxsum[blk];
                }
                const int4 w = wb[j];
                const int4 lo = make_int4(w.x & 0x0F0F0F0F, w.y & 0x0F0F0F0F, w.z & 0x0F0F0F0F, w.w & 0x0F0F0F0F);
                const int4 hi =
                    make_int4((int)(((uint32_t)w.x >> 4) & 0x0F0F0F0Fu), (int)(((uint32_t)w.y >> 4) & 0x0F0F0F0Fu),
                              (int)(((uint32_t)w.z >> 4) & 0x0F0F0F0Fu), (int)(((uint32_t)w.w >> 4) & 0x0F0F0F0Fu));
                // nibble j is w_j + 8: sum_b = Σ lo·x_j + Σ hi·x_j+16 - 8·Σ x
                const int s = dot16(hi, x1, dot16(lo, x0, 0)) - 8 * xsum;
                t = (float)s * (sb[j] * xsv);
                // block 64pc+l is in lane l; running sum L (lane L) takes
                // lanes L, L+8, ..., L+56.
                float tj[8];
                tj[0] = t;
#pragma unroll
                for (int k = 1; k < 8; ++k) tj[k] = __shfl_down(t, 8 * k);
                if (lane < 8) {
#pragma unroll
                    for (int k = 0; k < 8; ++k)
                        if (pc * 64 + lane + 8 * k < nb) acc += tj[k];
                }
            }
            if (++pc == C) {
                float res;
                if (FMT == kFmtQ8) {
                    const float p2 = acc + __shfl_down(acc, 2);
                    const float q4 = p2 + __shfl_down(p2, 4);
                    res = q4 + __shfl_down(q4, 8);
                } else {
                    const float p2 = acc + __shfl_down(acc, 1);
                    const float q4 = p2 + __shfl_down(p2, 2);
                    res = q4 + __shfl_down(q4, 4);
                }
                if (lane == 0) epilogue(row_of(pp, ph), res);
                acc = 0.0f;
                pc = 0;
                next_row(pp, ph);
            }
        };

        for (int st = 0; st < nsteps; st += U) {
#pragma unroll
            for (int j = 0; j < U; j++) {
                if (st + j < nsteps) process(j);
                load(j);
            }
        }

        // ---- (5) the workgroup's results, coalesced ----
        __syncthreads();
        if (EPI == kEpSilu) {
            const int np = n >> 1, P0 = R0 >> 1;
            for (int i = threadIdx.x; i < np; i += NT) a.seg[0].out[P0 + i] = sres[i];
            if (a.qx_out) {
                // h's Q8_0 blocks: the launcher gives each workgroup whole
                // blocks (pairs in multiples of 32), eight lanes a block
                for (int g0 = 0; g0 < (np >> 2); g0 += NT) {  // uniform
                    const int g = g0 + threadIdx.x;
                    const int gc = min(g, (np >> 2) - 1);
                    const float4 v = reinterpret_cast<const float4 *>(sres)[gc];
                    float d;
                    int cs;
                    const uint32_t pk = quantize_group(v.x, v.y, v.z, v.w, d, cs);
                    if (g < (np >> 2)) {
                        reinterpret_cast<uint32_t *>(a.qx_out + P0)[g] = pk;
                        if ((g & 7) == 0) {
                            a.xs_out[(P0 >> 5) + (g >> 3)] = d;
                            a.xsum_out[(P0 >> 5) + (g >> 3)] = cs;
                        }
                    }
                }
            }
        } else if (EPI == kEpQKV) {
            for (int i = threadIdx.x; i < n; i += NT) {
                const int lg = a.row_base + R0 + i;
                float *dst = lg < a.qdim             ? a.seg[0].out + lg
                             : lg < a.qdim + a.kvdim ? a.kcache + (int64_t)pos * a.kvdim + (lg - a.qdim)
                                                     : a.vcache + (int64_t)pos * a.kvdim + (lg - a.qdim - a.kvdim);
                *dst = sres[i];
            }
        } else {
            for (int i = threadIdx.x; i < n; i += NT) {
                const RowSrc rs = row_src<EPI>(a, R0 + i, rowbytes, nb);
                rs.out[rs.r] = sres[i];
            }
        }
    }

    if (EPI == kEpLogits && work) {
        // Greedy argmax: per wave, per workgroup, then one atomicMax of the
        // workgroup's key into a slot (launch_advance folds the slots).
        if (lane == 0) {
            s_wv[wave] = best_v;
            s_wi[wave] = best_i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float bv = 0.0f;
            int bi = -1;
            for (int w = 0; w < W; w++) argmax_merge(bv, bi, s_wv[w], s_wi[w]);
            unsigned long long key = bi < 0 ? 0ull : argmax_key(bv, bi);
            // A NaN first logit makes the argmax 0 (nothing compares above
            // it): the largest key, row 0.
            if (R0 == 0 && sres[0] != sres[0]) key = ~0ull;
            if (key) atomicMax(&a.amax[blockIdx.x % kArgmaxSlots], key);
        }
    }
}

// ---------------------------------------------------------------------------
// Launch: the host sizes the grid (about two workgroups per CU, rows split
// evenly, pairs kept whole) and the LDS layout.

// Chunks in flight per wave: 2 when the input comes quantized, 4 to cover
// an LDS prologue (measured; 6 under the RMSNorm prologue measured slower).
template <int FMT, int PRO, int EPI, int W>
static void launch_one(const FusedArgs &a, unsigned grid, size_t lds, hipStream_t s) {
    RK_LAUNCH((fused_kernel<FMT, PRO, EPI, W, PRO == kProGlobal ? 2 : 4>), dim3(grid), dim3(64 * W), lds, s, a);
}

template <int FMT, int PRO, int W>
static bool launch_epi(int epi, const FusedArgs &a, unsigned grid, size_t lds, hipStream_t s) {
    switch (epi) {
        case kEpStore: launch_one<FMT, PRO, kEpStore, W>(a, grid, lds, s); return true;
        case kEpAdd: launch_one<FMT, PRO, kEpAdd, W>(a, grid, lds, s); return true;
        case kEpAddCanon: launch_one<FMT, PRO, kEpAddCanon, W>(a, grid, lds, s); return true;
        case kEpQKV: launch_one<FMT, PRO, kEpQKV, W>(a, grid, lds, s); return true;
        case kEpSilu: launch_one<FMT, PRO, kEpSilu, W>(a, grid, lds, s); return true;
        case kEpLogits: launch_one<FMT, PRO, kEpLogits, W>(a, grid, lds, s); return true;
    }
    return false;
}

template <int FMT, int W>
static bool launch_pro(int pro, int epi, const FusedArgs &a, unsigned grid, size_t lds, hipStream_t s) {
    switch (pro) {
        case kProGlobal: return launch_epi<FMT, kProGlobal, W>(epi, a, grid, lds, s);
        case kProQuant: return launch_epi<FMT, kProQuant, W>(epi, a, grid, lds, s);
        case kProNorm: return launch_epi<FMT, kProNorm, W>(epi, a, grid, lds, s);
    }
    return false;
}

static inline int align16(int v) { return (v + 15) & ~15; }

// Dynamic LDS a launch may ask for without raising the kernel's limit.
constexpr int kMaxDynLds = 64 * 1024;

static void lds_layout(FusedArgs &a, int pro, int epi) {
    const int cols = a.cols, nb = cols >> 5;
    int at = 0;
    if (pro != kProGlobal) {
        a.lds_xs = align16(cols);
        a.lds_xsum = a.lds_xs + align16(nb * 4);
        at = a.lds_xsum + align16(nb * 4);
    }
    if (pro == kProNorm) {  // x transposed for Dot32 (wg_norm_quant)
        a.lds_norm = at;
        at += (int)norm_lds(cols);
    }
    a.lds_res = at;
    at += align16(a.rows_per_wg * 4);
    a.lds_ep = at;
    if (epi != kEpSilu && epi != kEpLogits) at += align16(a.rows_per_wg * 4 + (epi == kEpQKV ? 4 * a.hs : 0));
    a.lds_bytes = at;
}

// Rows per workgroup at most: per-row operands are loaded one per thread of
// the smallest workgroup, and results wait in LDS.
constexpr int kMaxRowsPerWg = 512;

bool fused_fits(int pro, int cols) {
    if (cols <= 0 || cols % 32 != 0) return false;
    if (pro == kProGlobal) return true;
    if (cols > (pro == kProNorm ? kMaxNormProCols : kMaxLdsCols)) return false;
    FusedArgs a{};
    a.cols = cols;
    a.rows_per_wg = kMaxRowsPerWg;
    a.hs = 1024;
    lds_layout(a, pro, kEpQKV);
    return a.lds_bytes <= kMaxDynLds;
}

bool launch_fused(int fmt, int pro, int epi, FusedArgs a, int cu, hipStream_t s) {
    if (a.rows <= 0) return true;
    if (launch_stream(fmt, pro, epi, a, cu, s)) return true;
    if (!fused_fits(pro, a.cols)) return false;
    if ((epi == kEpAdd || epi == kEpAddCanon || epi == kEpLogits) && a.nseg != 1) return false;
    if (epi == kEpQKV && (a.hs <= 0 || a.hs > 1024 || (a.rows & 1) || (a.row_base & 1))) return false;
    const bool pair = epi == kEpQKV || epi == kEpSilu;
    // Workgroup shape (measured on MI355X): with the input already
    // quantized, 8 waves x 2 workgroups per CU, or 16 waves x 1 for mid-size
    // row counts; with an LDS prologue, 16 waves x 1 up to 8192 rows, else
    // 8 x 2.
    const int64_t ncu = cu > 0 ? cu : 256;
    bool w16;
    int per_cu;
    if (pro == kProGlobal) {
        w16 = a.rows > 5000 && a.rows < 20000;
        per_cu = w16 ? 1 : 2;
    } else {  // an LDS prologue (quantize, or RMSNorm and quantize)
        w16 = a.rows <= 8192;
        per_cu = w16 ? 1 : 2;
    }
    const int64_t target = ncu * per_cu;
    int64_t rpw = (a.rows + target - 1) / target;
    if (rpw > kMaxRowsPerWg) rpw = kMaxRowsPerWg;
    if (pair) rpw = (rpw + 1) & ~(int64_t)1;
    if (epi == kEpSilu && a.qx_out) {
        // whole Q8 blocks of h per workgroup: 64 interleaved rows (32 of h)
        // each, as many workgroups as that gives (rounding up to 128 rows
        // left too few workgroups to keep the weight stream busy)
        if (a.rows % 64 != 0) return false;
        rpw = 64;
    }
    a.rows_per_wg = (int32_t)rpw;
    const unsigned grid = (unsigned)((a.rows + rpw - 1) / rpw);
    lds_layout(a, pro, epi);
    const size_t lds = (size_t)a.lds_bytes;
    if (lds > (size_t)kMaxDynLds) return false;
    if (fmt == kFmtQ8)
        return w16 ? launch_pro<kFmtQ8, 16>(pro, epi, a, grid, lds, s) : launch_pro<kFmtQ8, 8>(pro, epi, a, grid, lds, s);
    return w16 ? launch_pro<kFmtQ4, 16>(pro, epi, a, grid, lds, s) : launch_pro<kFmtQ4, 8>(pro, epi, a, grid, lds, s);
}

// ---------------------------------------------------------------------------
// Attention of the position ctl[kCtlPos] (internal/llm/model.go:575-591).

// Scores: score_t = float32(Dot32(q_h, k_t)·invSqrt) for t <= position.
// Four lanes (a quad) per position, 64 positions per workgroup, grid
// (heads, position tiles); tiles past the position exit. Lane `sub` of the
// quad keeps Dot32's running sums j = 8·sub .. 8·sub+7 (element i goes to
// sum i mod 32, in order of i); the quad then forms e_j = (s_j + s_j+8) +
// (s_j+16 + s_j+24) by two DPP exchanges and lane 0 the final tree.
constexpr int kScoreTile = 64;

// Dot32(q_h, k_t) of head size hs (a multiple of 8; all loads issued at once
// when hs is a compile-time constant) by the quad of lanes `sub` = lane & 3:
// the result is in the quad's lane 0.
__device__ __forceinline__ float quad_dot32(const float *qh, const float *kt, int sub, int hs) {
    float s[8];
#pragma unroll
    for (int k = 0; k < 8; k++) s[k] = 0.0f;
    for (int base = 8 * sub; base < hs; base += 32) {
        const float4 k0 = *reinterpret_cast<const float4 *>(kt + base);
        const float4 k1 = *reinterpret_cast<const float4 *>(kt + base + 4);
        const float4 q0 = *reinterpret_cast<const float4 *>(qh + base);
        const float4 q1 = *reinterpret_cast<const float4 *>(qh + base + 4);
        s[0] += q0.x * k0.x;
        s[1] += q0.y * k0.y;
        s[2] += q0.z * k0.z;
        s[3] += q0.w * k0.w;
        s[4] += q1.x * k1.x;
        s[5] += q1.y * k1.y;
        s[6] += q1.z * k1.z;
        s[7] += q1.w * k1.w;
    }
    float e[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float u = s[k] + dppf_x1(s[k]);  // lane 0: s_j + s_j+8; lane 2: s_j+16 + s_j+24
        e[k] = u + dppf_x2(u);                 // lane 0: e_j
    }
    return ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
}

template <int HS>  // head size when fixed at compile time (all loads issued at once), else 0
__global__ __launch_bounds__(256) void att_scores_kernel(const float *q, const float *keys, float *att,
                                                         int32_t att_stride, const int32_t *ctl, AttBatch bt,
                                                         int kv_mul, int hs_rt, int kv_dim, float inv_sqrt) {
    const int hs = HS ? HS : hs_rt;
    const int z = blockIdx.z;  // token of a batch (0 when the position comes from ctl)
    const int T = att_position(ctl, bt, z) + 1;
    q += (int64_t)z * bt.q_stride;
    att += (int64_t)z * bt.att_stride;
    keys += (int64_t)z * bt.cache_stride;
    const int t0 = blockIdx.y * kScoreTile;
    if (t0 >= T) return;
    const int h = blockIdx.x, g = h / kv_mul;
    const int sub = threadIdx.x & 3;
    const int t = t0 + (threadIdx.x >> 2);
    const bool valid = t < T;
    const float *kt = keys + (int64_t)(valid ? t : t0) * kv_dim + (int64_t)g * hs;
    const float *qh = q + (int64_t)h * hs;
    float dot;
    if ((hs & 7) == 0 && (kv_dim & 3) == 0) {
        dot = quad_dot32(qh, kt, sub, hs);
    } else {
        float s[8];
#pragma unroll
        for (int k = 0; k < 8; k++) s[k] = 0.0f;
        for (int base = 8 * sub; base < hs; base += 32)
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (base + k < hs) s[k] += qh[base + k] * kt[base + k];
        float e[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float u = s[k] + dppf_x1(s[k]);
            e[k] = u + dppf_x2(u);
        }
        dot = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
    }
    if (sub == 0 && valid) att[(int64_t)h * att_stride + t] = dot * inv_sqrt;
}

void launch_att_scores(const float *q, const float *keys, float *att, int32_t att_stride, const int32_t *ctl,
                       const AttBatch &bt, int ctx, int heads, int kv_heads, int hs, int kv_dim, float inv_sqrt,
                       hipStream_t s) {
    if (!ctl && hs == 128 && att_group_fits(bt, hs, kv_dim)) {
        launch_att_scores_group(q, keys, att, att_stride, bt, heads, kv_heads, kv_dim, inv_sqrt, s);
        return;
    }
    // decode and independent sequences: positions up to ctx (tiles past a
    // token's position exit); a batch: up to its last token's
    const int npos = ctl || bt.pos ? ctx : bt.pos0 + bt.tokens;
    const dim3 grid(heads, (npos + kScoreTile - 1) / kScoreTile, ctl ? 1 : bt.tokens);
    if (hs == 128)
        RK_LAUNCH(att_scores_kernel<128>, grid, dim3(256), 0, s, q, keys, att, att_stride, ctl, bt, heads / kv_heads,
                  hs, kv_dim, inv_sqrt);
    else
        RK_LAUNCH(att_scores_kernel<0>, grid, dim3(256), 0, s, q, keys, att, att_stride, ctl, bt, heads / kv_heads, hs,
                  kv_dim, inv_sqrt);
}

// QK-norm and RoPE of one head by one wave: dst = RoPE_pos(w·(Rsqrt32(ss)·x))
// with ss = Dot32(x, x)·recip_hs + eps; pair (2p, 2p+1) rotated by table
// entry p. dst may be x (each lane reads its pairs before writing them, and
// the dot is complete before any write).
__device__ __forceinline__ void qk_norm_rope_wave(const float *x, const float *w, float recip_hs, float eps,
                                                  const float *cos_t, const float *sin_t, int pos, int hs,
                                                  float *dst) {
    const int lane = threadIdx.x & 63;
    const float dot = __shfl(dot32_half(x, x, hs, lane & 31, lane < 32), 0);
    const float r = rsqrt32((dot * recip_hs) + eps);
    const int half = hs >> 1;
    for (int p = lane; p < half; p += 64) {
        const float co = cos_t[(int64_t)pos * half + p], si = sin_t[(int64_t)pos * half + p];
        const float v0 = w[2 * p] * (r * x[2 * p]), v1 = w[2 * p + 1] * (r * x[2 * p + 1]);
        dst[2 * p] = (v0 * co) - (v1 * si);
        dst[2 * p + 1] = (v0 * si) + (v1 * co);
    }
}

// qk_norm_rope_wave's steps for hs = 128 on inputs loaded ahead into
// registers (qk_row_load, issued before other loads so that the norm waits
// only for its own): lane l < 32 keeps x_l, x_l+32, x_l+64, x_l+96 for the
// Dot32 running sum l; lane p the pair (2p, 2p+1), its weights and table
// entry p.
struct QkRow {
    float d[4], x0, x1, w0, w1, co, si;
};

__device__ __forceinline__ void qk_row_load(const float *x, const float *w, const float *cos_t, const float *sin_t,
                                            int pos, QkRow &r) {
    const int lane = threadIdx.x & 63, hl = lane & 31;
#pragma unroll
    for (int k = 0; k < 4; k++) r.d[k] = x[hl + 32 * k];
    r.x0 = x[2 * lane];
    r.x1 = x[2 * lane + 1];
    r.w0 = w[2 * lane];
    r.w1 = w[2 * lane + 1];
    r.co = cos_t[(int64_t)pos * 64 + lane];
    r.si = sin_t[(int64_t)pos * 64 + lane];
}

__device__ __forceinline__ void qk_row_norm_rope(const QkRow &r, float recip_hs, float eps, float *dst) {
    const int lane = threadIdx.x & 63;
    float s = 0.0f;
    if (lane < 32) {
#pragma unroll
        for (int k = 0; k < 4; k++) s += r.d[k] * r.d[k];
    }
    const float dot = __shfl(dot32_reduce(s), 0);
    const float rr = rsqrt32((dot * recip_hs) + eps);
    const float v0 = r.w0 * (rr * r.x0), v1 = r.w1 * (rr * r.x1);
    dst[2 * lane] = (v0 * r.co) - (v1 * r.si);
    dst[2 * lane + 1] = (v0 * r.si) + (v1 * r.co);
}

// The scores of a decode step (or of independent sequences) with the
// QK-norm and RoPE of the position's q and k folded in: wave 0 normalizes
// the workgroup's q head into LDS, wave 1 (in the tile that holds the
// position) the key of its kv head; the position's own score takes that key
// from LDS, and one workgroup per kv head stores it and the raw v into the
// caches (read by the values launch that follows). q_raw, k_raw, v_raw: the
// token's QKV outputs, [tokens][heads·hs] and [tokens][kv_dim]. hs: a
// multiple of 8, at most kQknMaxHs.
constexpr int kQknMaxHs = 256;
// HS: the head size when it is 128 (the keys of the workgroup's positions
// then load into registers before the norm, so the dots wait on LDS only),
// else 0 (the keys read at the dots).
template <int HS>
__global__ __launch_bounds__(256) void att_scores_qkn_kernel(const float *q_raw, const float *k_raw, const float *v_raw,
                                                             const float *q_norm, const float *k_norm, float recip_hs,
                                                             float eps, const float *cos_t, const float *sin_t,
                                                             float *keys, float *vals, float *att, int32_t att_stride,
                                                             const int32_t *ctl, AttBatch bt, int kv_mul, int hs,
                                                             int kv_dim, float inv_sqrt) {
    __shared__ __align__(16) float sq[kQknMaxHs], sk[kQknMaxHs];
    const int z = blockIdx.z;
    const int pos = att_position(ctl, bt, z), T = pos + 1;
    const int t0 = blockIdx.y * kScoreTile;
    if (t0 >= T) return;
    const int heads = gridDim.x;
    q_raw += (int64_t)z * heads * hs;
    k_raw += (int64_t)z * kv_dim;
    v_raw += (int64_t)z * kv_dim;
    att += (int64_t)z * bt.att_stride;
    keys += (int64_t)z * bt.cache_stride;
    vals += (int64_t)z * bt.cache_stride;
    const int h = blockIdx.x, g = h / kv_mul;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool here = pos < t0 + kScoreTile;  // the tile holds the position
    const int sub = threadIdx.x & 3;
    const int t = t0 + (threadIdx.x >> 2);
    // HS = 128: this lane's part of its position's key (the position's own
    // row is taken from LDS below; its cache row is read here and dropped)
    float4 kr[HS ? HS / 32 : 1][2];
    if (HS) {
        const float *kg = keys + (int64_t)(t < T ? t : t0) * kv_dim + (int64_t)g * hs + 8 * sub;
#pragma unroll
        for (int it = 0; it < (HS ? HS / 32 : 1); it++) {
            kr[it][0] = *reinterpret_cast<const float4 *>(kg + 32 * it);
            kr[it][1] = *reinterpret_cast<const float4 *>(kg + 32 * it + 4);
        }
    }
    if (wave == 0)
        qk_norm_rope_wave(q_raw + (int64_t)h * hs, q_norm, recip_hs, eps, cos_t, sin_t, pos, hs, sq);
    else if (wave == 1 && here)
        qk_norm_rope_wave(k_raw + (int64_t)g * hs, k_norm, recip_hs, eps, cos_t, sin_t, pos, hs, sk);
    __syncthreads();
    if (here && h % kv_mul == 0 && wave == 2) {
        float *kd = keys + (int64_t)pos * kv_dim + (int64_t)g * hs;
        float *vd = vals + (int64_t)pos * kv_dim + (int64_t)g * hs;
        const float *vs = v_raw + (int64_t)g * hs;
        for (int i = lane; i < hs; i += 64) {
            kd[i] = sk[i];
            vd[i] = vs[i];
        }
    }
    float dot;
    if (HS) {
        if (t == pos) {
#pragma unroll
            for (int it = 0; it < (HS ? HS / 32 : 1); it++) {
                kr[it][0] = *reinterpret_cast<const float4 *>(sk + 8 * sub + 32 * it);
                kr[it][1] = *reinterpret_cast<const float4 *>(sk + 8 * sub + 32 * it + 4);
            }
        }
        // quad_dot32's steps on the held key
        float sacc[8];
#pragma unroll
        for (int k = 0; k < 8; k++) sacc[k] = 0.0f;
#pragma unroll
        for (int it = 0; it < (HS ? HS / 32 : 1); it++) {
            const float4 q0 = *reinterpret_cast<const float4 *>(sq + 8 * sub + 32 * it);
            const float4 q1 = *reinterpret_cast<const float4 *>(sq + 8 * sub + 32 * it + 4);
            sacc[0] += q0.x * kr[it][0].x;
            sacc[1] += q0.y * kr[it][0].y;
            sacc[2] += q0.z * kr[it][0].z;
            sacc[3] += q0.w * kr[it][0].w;
            sacc[4] += q1.x * kr[it][1].x;
            sacc[5] += q1.y * kr[it][1].y;
            sacc[6] += q1.z * kr[it][1].z;
            sacc[7] += q1.w * kr[it][1].w;
        }
        float e[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float u = sacc[k] + dppf_x1(sacc[k]);
            e[k] = u + dppf_x2(u);
        }
        dot = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
    } else {
        const float *kt = t == pos ? sk : keys + (int64_t)(t < T ? t : t0) * kv_dim + (int64_t)g * hs;
        dot = quad_dot32(sq, kt, sub, hs);
    }
    if (sub == 0 && t < T) att[(int64_t)h * att_stride + t] = dot * inv_sqrt;
}

bool launch_att_scores_qkn(const float *q_raw, const float *k_raw, const float *v_raw, const float *q_norm,
                           const float *k_norm, float recip_hs, float eps, const float *cos_t, const float *sin_t,
                           float *keys, float *vals, float *att, int32_t att_stride, const int32_t *ctl,
                           const AttBatch &bt, int ctx, int heads, int kv_heads, int hs, int kv_dim, float inv_sqrt,
                           hipStream_t s) {
    if (!ctl && !bt.pos) return false;  // a prompt's batch: the grouped scores, after the norm launch
    if (hs % 8 != 0 || hs > kQknMaxHs || kv_dim % 4 != 0 || kv_dim != kv_heads * hs) return false;
    const dim3 grid(heads, (ctx + kScoreTile - 1) / kScoreTile, ctl ? 1 : bt.tokens);
    if (hs == 128)
        RK_LAUNCH(att_scores_qkn_kernel<128>, grid, dim3(256), 0, s, q_raw, k_raw, v_raw, q_norm, k_norm, recip_hs, eps,
                  cos_t, sin_t, keys, vals, att, att_stride, ctl, bt, heads / kv_heads, hs, kv_dim, inv_sqrt);
    else
        RK_LAUNCH(att_scores_qkn_kernel<0>, grid, dim3(256), 0, s, q_raw, k_raw, v_raw, q_norm, k_norm, recip_hs, eps,
                  cos_t, sin_t, keys, vals, att, att_stride, ctl, bt, heads / kv_heads, hs, kv_dim, inv_sqrt);
    return true;
}

// Softmax and weighted values for a 32-element slice of one head per
// workgroup (grid: heads, ceil(hs/32)). The order is the CPU's: Go max,
// e_t = Exp32(s_t - max), one sequential sum, inv = Recip32(sum), a_t =
// e_t·inv, then out_i = Σ_t a_t·v_t,i in t order from +0. The slice's values
// for a chunk of positions are loaded up front (the first chunk's during the
// softmax, each next one's during the previous chunk's sums); a thread takes
// four consecutive positions of four elements, so the products a_t·v_t,i go
// to LDS transposed as 16-byte writes, and each element's sequential sum
// (wave 0, one lane per element) reads them four at a time. The product
// tiles are double-buffered: the other waves write chunk c+1's while wave 0
// sums chunk c. A slice holding a whole Q8 block is quantized for the next
// product. The LDS can exceed 64 KiB (gfx950 gives a workgroup 160 KiB).
// CH positions a chunk: 256, or 128 for contexts of up to 256 positions
// (half the LDS: four workgroups a CU, for many short sequences at once).
constexpr int kValSlice = 32;
constexpr int kValThreads = 256;
constexpr int kValChunk = 256;
constexpr int kValShortChunk = 128;
constexpr int kValShortCtx = 256;
// floats per element row of a product tile (an odd count of 16-byte units)
constexpr int val_pitch(int ch) { return ch + 4; }
// thread -> float4 column fq (elements 4fq..4fq+3) and position quad pq
// (positions 4pq..4pq+3 of a round); rounds cover the chunk
constexpr int kValQuads = kValThreads / (kValSlice / 4);             // position quads per round

// VEC: head size and value-row stride are multiples of 4, so a thread's four
// elements are one 16-byte load (a separate instance: a run-time choice would
// be if-converted into four 4-byte loads for every shape).
//
// The body for head bh, slice by and token z; SIG as att_values_reg_body's
// (the Q8_0 block handed to the Wo workgroups of att_values_wo_kernel).
// QKN (a decode step, hs = 128, contexts up to 256; qk given): the scores
// are formed here from the raw q and k rows (att_scores_qkn_kernel's
// steps: QK-norm and RoPE of q's head and of the position's key into LDS,
// each cached key of the kv head read by a quad of lanes at the start),
// one workgroup per kv head stores the position's k and v into the caches,
// and the position's own value row is read from v_raw (no workgroup of
// the launch reads the caches at the position).
template <bool VEC, int CH, bool SIG, bool QKN = false>
__device__ __forceinline__ void att_values_body(const float *att, int32_t att_stride, const float *vals, float *out,
                                                const int32_t *ctl, const AttBatch &bt, int kv_mul, int hs,
                                                int kv_dim, int ctx_pad, int8_t *qx, float *xs, int32_t *xsum, int bh,
                                                int by, int z, unsigned long long *sync, int na,
                                                const QknIn *qk = nullptr) {
    extern __shared__ __align__(16) float smem[];
    __shared__ float s_red[kValThreads / 64];
    __shared__ float s_inv;
    __shared__ __align__(16) float s_res[kValSlice];
    float *sa = smem;            // [ctx_pad] scores -> weights
    constexpr int kValPitch = val_pitch(CH), kValRounds = CH / (4 * kValQuads);
    static_assert(kValRounds >= 1, "a chunk is whole rounds");
    float *sp = smem + ctx_pad;  // [2][kValSlice][kValPitch] product tiles of two chunks
    const int T = att_position(ctl, bt, z) + 1;
    att += (int64_t)z * bt.att_stride;
    out += (int64_t)z * bt.out_stride;
    vals += (int64_t)z * bt.cache_stride;
    if (qx) {
        qx += (int64_t)z * bt.out_stride;
        xs += (int64_t)z * (bt.out_stride >> 5);
        xsum += (int64_t)z * (bt.out_stride >> 5);
    }
    const int h = bh, g = h / kv_mul;
    const int e0 = by * kValSlice;
    const int ne = min(kValSlice, hs - e0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *vbase = vals + (int64_t)g * hs + e0;
    const int fq = tid & 7, pq = tid >> 3;

    // One chunk of values in registers, loaded during the softmax (the
    // first) or the previous chunk's sums. Loads are unconditional (position
    // clamped to T-1, element column to the slice): values past T or the
    // slice give products that are never summed or output.
    float4 vr[kValRounds][4];  // [round][position within the quad]
    auto load_chunk = [&](int c0) {
#pragma unroll
        for (int r = 0; r < kValRounds; r++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int t = min(c0 + 4 * (pq + kValQuads * r) + j, T - 1);
                const float *row =
                    QKN && t == T - 1 ? qk->v_raw + (int64_t)g * hs + e0 : vbase + (int64_t)t * kv_dim;
                if (VEC) {
                    vr[r][j] = *reinterpret_cast<const float4 *>(row + min(4 * fq, ne - 4));
                } else {
                    vr[r][j].x = row[min(4 * fq, ne - 1)];
                    vr[r][j].y = row[min(4 * fq + 1, ne - 1)];
                    vr[r][j].z = row[min(4 * fq + 2, ne - 1)];
                    vr[r][j].w = row[min(4 * fq + 3, ne - 1)];
                }
            }
        }
    };
    // the head's scores (the first 1024 with the values, all in flight)
    const float *ah = att + (int64_t)h * att_stride;
    constexpr int kScPer = 1024 / kValThreads;
    float sv[kScPer];
    if (QKN) {
        static_assert(!QKN || (CH == kValShortChunk && kValThreads == 256), "QKN: the short form");
        __shared__ __align__(16) float sq[128], sk[128];
        const int pos = T - 1, sub = tid & 3;
        // waves 0 and 1: q's head and the position's key, requested first
        QkRow qr;
        if (wave == 0)
            qk_row_load(qk->q_raw + (int64_t)h * 128, qk->q_norm, qk->cos_t, qk->sin_t, pos, qr);
        else if (wave == 1)
            qk_row_load(qk->k_raw + (int64_t)g * 128, qk->k_norm, qk->cos_t, qk->sin_t, pos, qr);
        // lane sub of position t: elements 8·sub + 32·it + 0..7 of its key
        auto load_key = [&](int t, float4 (&kr)[4][2]) {
            const float *kg = qk->keys + (int64_t)(t < T ? t : 0) * kv_dim + (int64_t)g * 128 + 8 * sub;
#pragma unroll
            for (int it = 0; it < 4; it++) {
                kr[it][0] = *reinterpret_cast<const float4 *>(kg + 32 * it);
                kr[it][1] = *reinterpret_cast<const float4 *>(kg + 32 * it + 4);
            }
        };
        // Dot32(q, k_t)·inv_sqrt on the held key (quad_dot32's steps; the
        // position's own key from LDS), valid in the quad's lane 0
        auto score = [&](int t, float4 (&kr)[4][2]) -> float {
            if (t == pos) {
#pragma unroll
                for (int it = 0; it < 4; it++) {
                    kr[it][0] = *reinterpret_cast<const float4 *>(sk + 8 * sub + 32 * it);
                    kr[it][1] = *reinterpret_cast<const float4 *>(sk + 8 * sub + 32 * it + 4);
                }
            }
            float sacc[8];
#pragma unroll
            for (int k = 0; k < 8; k++) sacc[k] = 0.0f;
#pragma unroll
            for (int it = 0; it < 4; it++) {
                const float4 q0 = *reinterpret_cast<const float4 *>(sq + 8 * sub + 32 * it);
                const float4 q1 = *reinterpret_cast<const float4 *>(sq + 8 * sub + 32 * it + 4);
                sacc[0] += q0.x * kr[it][0].x;
                sacc[1] += q0.y * kr[it][0].y;
                sacc[2] += q0.z * kr[it][0].z;
                sacc[3] += q0.w * kr[it][0].w;
                sacc[4] += q1.x * kr[it][1].x;
                sacc[5] += q1.y * kr[it][1].y;
                sacc[6] += q1.z * kr[it][1].z;
                sacc[7] += q1.w * kr[it][1].w;
            }
            float e[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float u = sacc[k] + dppf_x1(sacc[k]);
                e[k] = u + dppf_x2(u);
            }
            return (((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]))) * qk->inv_sqrt;
        };
        // positions in rounds of 64 (a quad each): two rounds' keys in
        // flight at the start, the rest (contexts past 128) after
        const int t0 = tid >> 2;
        float4 ka[4][2], kb[4][2];
        load_key(t0, ka);
        if (T > 64) load_key(t0 + 64, kb);  // uniform
        load_chunk(0);
        if (wave < 2) qk_row_norm_rope(qr, qk->recip_hs, qk->eps, wave == 0 ? sq : sk);
        __syncthreads();
        if (h % kv_mul == 0 && by == 0 && wave == 2) {
            // the kv head's first workgroup: the position's k and v into
            // the caches (read by the next launches)
            float *kd = qk->keys + (int64_t)pos * kv_dim + (int64_t)g * 128;
            float *vd = qk->vals + (int64_t)pos * kv_dim + (int64_t)g * 128;
            const float *vs = qk->v_raw + (int64_t)g * 128;
            for (int i = lane; i < 128; i += 64) {
                kd[i] = sk[i];
                vd[i] = vs[i];
            }
        }
        // the scores in registers (quad lane 0: position t0 + 64r), their
        // maximum (Go max, any order; -inf leaves it unchanged)
        float dsc[4];
        float m = -__builtin_huge_valf();
        dsc[0] = score(t0, ka);
        if (T > 64) dsc[1] = score(t0 + 64, kb);
        if (T > 128) {  // uniform
            load_key(t0 + 128, ka);
            if (T > 192) load_key(t0 + 192, kb);
            dsc[2] = score(t0 + 128, ka);
            if (T > 192) dsc[3] = score(t0 + 192, kb);
        }
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (sub == 0 && t0 + 64 * r < T) m = gomax(m, dsc[r]);
        m = wave_gomax(m);
        if (lane == 0) s_red[wave] = m;
        __syncthreads();
        m = s_red[0];
#pragma unroll
        for (int w = 1; w < kValThreads / 64; w++) m = gomax(m, s_red[w]);
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (sub == 0 && t0 + 64 * r < T) sa[t0 + 64 * r] = exp32(dsc[r] - m);
        __syncthreads();
    } else {
#pragma unroll
        for (int k = 0; k < kScPer; k++) sv[k] = ah[min(tid + kValThreads * k, T - 1)];
        load_chunk(0);
    }

    if (!QKN) {
        // softmax of the head's scores
        float m = sv[0];
#pragma unroll
        for (int k = 0; k < kScPer; k++) {
            if (tid + kValThreads * k < T) {
                sa[tid + kValThreads * k] = sv[k];
                m = gomax(m, sv[k]);
            }
        }
        for (int t = tid + kValThreads * kScPer; t < T; t += kValThreads) {
            const float v = ah[t];
            sa[t] = v;
            m = gomax(m, v);
        }
        m = wave_gomax(m);
        if (lane == 0) s_red[wave] = m;
        __syncthreads();
        m = s_red[0];
#pragma unroll
        for (int w = 1; w < kValThreads / 64; w++) m = gomax(m, s_red[w]);
        for (int t = tid; t < T; t += kValThreads) sa[t] = exp32(sa[t] - m);
        __syncthreads();
    }
    if (tid == 0) s_inv = recip32(lds_chain_sum(sa, T, 0.0f));
    __syncthreads();
    const float inv = s_inv;  // a_t = e_t·inv, formed where the products read e_t

    // Chunk c: its products into tile c mod 2, chunk c+1's loads, a barrier,
    // then wave 0's sums over the tile. The tile was last read by wave 0's
    // sums two chunks ago, which ended before it reached the previous barrier,
    // so the other waves write chunk c+1's products while wave 0 sums chunk c.
    float acc = 0.0f;
    int buf = 0;
    for (int c0 = 0; c0 < T; c0 += CH, buf ^= 1) {
        float *tile = sp + buf * (kValSlice * kValPitch);
#pragma unroll
        for (int r = 0; r < kValRounds; r++) {
            const int tt = 4 * (pq + kValQuads * r);
            const float4 e4 = *reinterpret_cast<const float4 *>(sa + min(c0 + tt, ctx_pad - 4));
            const float4 a4 = make_float4(e4.x * inv, e4.y * inv, e4.z * inv, e4.w * inv);
            float *dst = tile + (4 * fq) * kValPitch + tt;
            *reinterpret_cast<float4 *>(dst) =
                make_float4(a4.x * vr[r][0].x, a4.y * vr[r][1].x, a4.z * vr[r][2].x, a4.w * vr[r][3].x);
            *reinterpret_cast<float4 *>(dst + kValPitch) =
                make_float4(a4.x * vr[r][0].y, a4.y * vr[r][1].y, a4.z * vr[r][2].y, a4.w * vr[r][3].y);
            *reinterpret_cast<float4 *>(dst + 2 * kValPitch) =
                make_float4(a4.x * vr[r][0].z, a4.y * vr[r][1].z, a4.z * vr[r][2].z, a4.w * vr[r][3].z);
            *reinterpret_cast<float4 *>(dst + 3 * kValPitch) =
                make_float4(a4.x * vr[r][0].w, a4.y * vr[r][1].w, a4.z * vr[r][2].w, a4.w * vr[r][3].w);
        }
        load_chunk(c0 + CH);  // in flight while this chunk is summed
        __syncthreads();
        const int n = min(CH, T - c0);
        if (wave == 0 && lane < kValSlice) acc = lds_chain_sum(tile + lane * kValPitch, n, acc);
    }
    if (wave == 0 && lane < ne) out[(int64_t)h * hs + e0 + lane] = acc;
    if (qx && ne == kValSlice) {
        // the slice is one Q8_0 block of the next input (e0 is a multiple
        // of 32): lanes 0-7 of wave 0 take four values each, through a
        // buffer only wave 0 touches (no barrier)
        if (wave == 0) {
            if (lane < kValSlice) s_res[lane] = acc;
            const int q = min(lane, 7);
            const float4 v4 = reinterpret_cast<const float4 *>(s_res)[q];
            float d;
            int cs;
            const uint32_t pk = quantize_group(v4.x, v4.y, v4.z, v4.w, d, cs);
            const int64_t base = (int64_t)h * hs + e0;
            if (SIG) {
                // agent-scope stores, complete before the count
                if (lane < 8) {
                    __hip_atomic_store(reinterpret_cast<uint32_t *>(qx + base) + lane, pk, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                    if (lane == 0) {
                        __hip_atomic_store(xs + (base >> 5), d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        xsum[base >> 5] = cs;
                    }
                }
                sync_signal_done(sync, na);
            } else if (lane < 8) {
                reinterpret_cast<uint32_t *>(qx + base)[lane] = pk;
                if (lane == 0) {
                    xs[base >> 5] = d;
                    xsum[base >> 5] = cs;
                }
            }
        }
    }
}

template <bool VEC, int CH>
__global__ __launch_bounds__(kValThreads) void att_values_kernel(const float *att, int32_t att_stride,
                                                                 const float *vals, float *out, const int32_t *ctl,
                                                                 AttBatch bt, int kv_mul, int hs, int kv_dim,
                                                                 int ctx_pad, int8_t *qx, float *xs, int32_t *xsum) {
    att_values_body<VEC, CH, false>(att, att_stride, vals, out, ctl, bt, kv_mul, hs, kv_dim, ctx_pad, qx, xs, xsum,
                                    blockIdx.x, blockIdx.y, blockIdx.z, nullptr, 0);
}

// The same result for contexts up to kVrMaxCtx positions, with every
// position's values of the slice in registers from the start. Waves 0-3
// take the scores and the softmax as above (lane 0 of wave 0 adds the
// e_t); waves 4-7 load the slice's values of chunks of kVrChunk positions
// (two position quads of one float4 column a thread a chunk, loads only
// for chunks below T) and, once inv is known, write a chunk's products
// a_t·v_t,i transposed into a tile while wave 0 adds the previous chunk's
// (lane i < 32: its element's products in position order). Tile row i
// keeps logical float4 q of the row at q ^ vr_swz(i): with that swizzle
// both the products' 16-byte writes (eight lanes: eight rows 4 apart, one
// column) and the sums' reads (eight lanes: eight consecutive rows, one
// logical column) touch 32 distinct banks.
constexpr int kVrThreads = 512;
constexpr int kVrChunk = 256;
constexpr int kVrMaxChunks = 4;
constexpr int kVrMaxCtx = kVrChunk * kVrMaxChunks;

__device__ __forceinline__ int vr_swz(int i) { return ((i >> 2) ^ ((i & 3) << 1)) & 7; }

// acc + row[0] + ... + row[n-1] in order for a tile row with swizzle key
// `key` (logical float4 q at q ^ key), n <= kVrChunk: batches of 32 values,
// the next batch's reads in flight during the current batch's additions.
__device__ __forceinline__ void swz_load_batch(float4 (&b)[kChainBatch], const float4 *q, int key) {
#pragma unroll
    for (int k = 0; k < kChainBatch; k++) b[k] = q[k ^ key];
}

__device__ __forceinline__ float swz_chain_sum(const float *row, int n, int key, float acc) {
    const float4 *q = reinterpret_cast<const float4 *>(row);
    const int nb = n >> 5;
    if (nb > 0) {
        float4 a[kChainBatch], b[kChainBatch];
        swz_load_batch(a, q, key);
        int k = 1;
        for (; k + 1 < nb; k += 2) {
            swz_load_batch(b, q + k * kChainBatch, key);
            __builtin_amdgcn_sched_barrier(0);
            acc = add_batch(a, acc);
            __builtin_amdgcn_sched_barrier(0);
            swz_load_batch(a, q + (k + 1) * kChainBatch, key);
            __builtin_amdgcn_sched_barrier(0);
            acc = add_batch(b, acc);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (k < nb) {
            swz_load_batch(b, q + k * kChainBatch, key);
            __builtin_amdgcn_sched_barrier(0);
            acc = add_batch(a, acc);
            __builtin_amdgcn_sched_barrier(0);
            acc = add_batch(b, acc);
        } else {
            acc = add_batch(a, acc);
        }
    }
    for (int t = nb * 32; t < n; t += 4) {  // the last partial batch, a float4 at a time
        const int l = t >> 2;
        const float4 v = q[l ^ key];
        acc += v.x;
        if (t + 1 < n) acc += v.y;
        if (t + 2 < n) acc += v.z;
        if (t + 3 < n) acc += v.w;
    }
    return acc;
}

// The body of att_values_reg_kernel for workgroup bx of token z. SIG: the
// values launch that also runs the Wo product (att_values_wo_kernel): the
// slice's Q8_0 block is stored through to the device's coherence point and
// the workgroup then counts itself done in `sync` (sync_signal_done).
template <bool SIG>
__device__ __forceinline__ void att_values_reg_body(const float *att, int32_t att_stride, const float *vals,
                                                    float *out, const int32_t *ctl, const AttBatch &bt, int kv_mul,
                                                    int hs, int kv_dim, int nsl, int ctx_pad, int8_t *qx, float *xs,
                                                    int32_t *xsum, int bx, int z, unsigned long long *sync, int na) {
    extern __shared__ __align__(16) float smem[];
    __shared__ float s_red[4];
    __shared__ float s_inv;
    __shared__ __align__(16) float s_res[kValSlice];
    float *sa = smem;               // [ctx_pad] scores -> e_t
    float *tiles = smem + ctx_pad;  // [2][32][kVrChunk] products, swizzled rows
    const int T = att_position(ctl, bt, z) + 1;
    const int nch = (T + kVrChunk - 1) / kVrChunk;
    att += (int64_t)z * bt.att_stride;
    out += (int64_t)z * bt.out_stride;
    vals += (int64_t)z * bt.cache_stride;
    if (qx) {
        qx += (int64_t)z * bt.out_stride;
        xs += (int64_t)z * (bt.out_stride >> 5);
        xsum += (int64_t)z * (bt.out_stride >> 5);
    }
    const int h = bx / nsl, e0 = (bx % nsl) * kValSlice;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // waves 4-7: float4 column fq (elements 4fq..4fq+3) and position quads
    // pq, pq + 32 of each chunk
    const int u = tid - 256, fq = u & 7, pq = u >> 3;
    float4 vr[kVrMaxChunks][2][4];  // [chunk][quad][position in the quad]
    float sc[4];
    if (wave < 4) {
        const float *ah = att + (int64_t)h * att_stride;
#pragma unroll
        for (int k = 0; k < 4; k++) sc[k] = ah[min(tid + 256 * k, T - 1)];
        float m = sc[0];
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (tid + 256 * k < T) m = gomax(m, sc[k]);
        m = wave_gomax(m);
        if (lane == 0) s_red[wave] = m;
    } else {
        // positions past T-1 load T-1's values (their products are never summed)
        const float *vb = vals + (int64_t)(h / kv_mul) * hs + e0 + 4 * fq;
#pragma unroll
        for (int c = 0; c < kVrMaxChunks; c++)
            if (c < nch) {  // uniform
#pragma unroll
                for (int q = 0; q < 2; q++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int t = min(c * kVrChunk + 4 * (pq + 32 * q) + j, T - 1);
                        vr[c][q][j] = *reinterpret_cast<const float4 *>(vb + (int64_t)t * kv_dim);
                    }
            }
    }
    __syncthreads();
    if (wave < 4) {
        float m = s_red[0];
#pragma unroll
        for (int w = 1; w < 4; w++) m = gomax(m, s_red[w]);
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (tid + 256 * k < T) sa[tid + 256 * k] = exp32(sc[k] - m);
    }
    __syncthreads();
    if (tid == 0) s_inv = recip32(lds_chain_sum(sa, T, 0.0f));
    __syncthreads();
    const float inv = s_inv;

    // chunk c's products into tile c mod 2 (waves 4-7); positions past T
    // take a clamped weight and give products that are never summed
    auto products = [&](int c) {
        float *tile = tiles + (c & 1) * (kValSlice * kVrChunk);
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int qd = pq + 32 * q;  // the quad within the chunk
            const float4 e4 = *reinterpret_cast<const float4 *>(sa + min(c * kVrChunk + 4 * qd, ctx_pad - 4));
            const float4 a4 = make_float4(e4.x * inv, e4.y * inv, e4.z * inv, e4.w * inv);
            const float4(&v)[4] = vr[c][q];
            const float4 p[4] = {make_float4(a4.x * v[0].x, a4.y * v[1].x, a4.z * v[2].x, a4.w * v[3].x),
                                 make_float4(a4.x * v[0].y, a4.y * v[1].y, a4.z * v[2].y, a4.w * v[3].y),
                                 make_float4(a4.x * v[0].z, a4.y * v[1].z, a4.z * v[2].z, a4.w * v[3].z),
                                 make_float4(a4.x * v[0].w, a4.y * v[1].w, a4.z * v[2].w, a4.w * v[3].w)};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = 4 * fq + j;
                reinterpret_cast<float4 *>(tile + i * kVrChunk)[qd ^ vr_swz(i)] = p[j];
            }
        }
    };
    if (wave >= 4) products(0);
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < kVrMaxChunks; c++) {
        if (c < nch) {  // uniform
            if (wave == 0) {
                if (lane < kValSlice)
                    acc = swz_chain_sum(tiles + (c & 1) * (kValSlice * kVrChunk) + lane * kVrChunk,
                                        min(kVrChunk, T - c * kVrChunk), vr_swz(lane), acc);
            } else if (wave >= 4 && c + 1 < nch) {
                products(c + 1);
            }
            __syncthreads();
        }
    }
    if (wave != 0) return;
    if (lane < kValSlice) out[(int64_t)h * hs + e0 + lane] = acc;
    if (qx) {
        // the slice is one Q8_0 block of the next input: lanes 0-7 take
        // four values each
        if (lane < kValSlice) s_res[lane] = acc;
        const int q = min(lane, 7);
        const float4 v4 = reinterpret_cast<const float4 *>(s_res)[q];
        float d;
        int cs;
        const uint32_t pk = quantize_group(v4.x, v4.y, v4.z, v4.w, d, cs);
        const int64_t base = (int64_t)h * hs + e0;
        if (SIG) {
            // agent-scope stores (written through to where every XCD's
            // loads of that scope look), complete before the count
            if (lane < 8) {
                __hip_atomic_store(reinterpret_cast<uint32_t *>(qx + base) + lane, pk, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                if (lane == 0) {
                    __hip_atomic_store(xs + (base >> 5), d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    xsum[base >> 5] = cs;
                }
            }
            sync_signal_done(sync, na);
        } else if (lane < 8) {
            reinterpret_cast<uint32_t *>(qx + base)[lane] = pk;
            if (lane == 0) {
                xs[base >> 5] = d;
                xsum[base >> 5] = cs;
            }
        }
    }
}

__global__ __launch_bounds__(kVrThreads) void att_values_reg_kernel(const float *att, int32_t att_stride,
                                                                    const float *vals, float *out, const int32_t *ctl,
                                                                    AttBatch bt, int kv_mul, int hs, int kv_dim,
                                                                    int nsl, int ctx_pad, int8_t *qx, float *xs,
                                                                    int32_t *xsum) {
    att_values_reg_body<false>(att, att_stride, vals, out, ctl, bt, kv_mul, hs, kv_dim, nsl, ctx_pad, qx, xs, xsum,
                               blockIdx.x, blockIdx.y, nullptr, 0);
}

static size_t att_values_reg_lds(int ctx) { return (size_t)(((ctx + 3) & ~3) + 2 * kValSlice * kVrChunk) * 4; }

// Dynamic LDS of the values kernel for a context of ctx positions.
static size_t att_values_lds(int ctx, int ch) { return (size_t)(((ctx + 3) & ~3) + 2 * kValSlice * val_pitch(ch)) * 4; }

// Dynamic LDS the values kernel may ask for: the device's 160 KiB less
// room for its static LDS.
constexpr size_t kValMaxDynLds = kMaxLdsBytes - 1024;

int att_values_max_ctx() { return (int)(kValMaxDynLds / 4 - 2 * kValSlice * val_pitch(kValChunk)) & ~3; }

void launch_att_values(const float *att, int32_t att_stride, const float *vals, float *out, const int32_t *ctl,
                       const AttBatch &bt, int ctx, int heads, int kv_heads, int hs, int kv_dim, int8_t *qx,
                       float *xs, int32_t *xsum, hipStream_t s, int cu) {
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute((const void *)att_values_kernel<true, kValChunk>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kValMaxDynLds);
        (void)hipFuncSetAttribute((const void *)att_values_kernel<false, kValChunk>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kValMaxDynLds);
        (void)hipFuncSetAttribute((const void *)att_values_reg_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)att_values_reg_lds(kVrMaxCtx));
    });
    if (!ctl && att_group_fits(bt, hs, kv_dim)) {
        launch_att_values_group(att, att_stride, vals, out, bt, heads, kv_heads, hs, kv_dim, qx, xs, xsum, s, cu);
        return;
    }
    if (hs % 32 != 0) qx = nullptr;
    const dim3 grid(heads, (hs + kValSlice - 1) / kValSlice, ctl ? 1 : bt.tokens);
    const int ctx_pad = (ctx + 3) & ~3;
    const bool vec = hs % 4 == 0 && kv_dim % 4 == 0;
    if (ctx <= kValShortCtx) {
        // short contexts: 128-position chunks (a third of the LDS, four
        // workgroups a CU); up to one chunk, one tile (eight a CU)
        const size_t lds = ctx <= kValShortChunk
                               ? (size_t)(ctx_pad + kValSlice * val_pitch(kValShortChunk)) * 4
                               : att_values_lds(ctx, kValShortChunk);
        if (vec)
            RK_LAUNCH((att_values_kernel<true, kValShortChunk>), grid, dim3(kValThreads), lds, s, att, att_stride, vals,
                      out, ctl, bt, heads / kv_heads, hs, kv_dim, ctx_pad, qx, xs, xsum);
        else
            RK_LAUNCH((att_values_kernel<false, kValShortChunk>), grid, dim3(kValThreads), lds, s, att, att_stride,
                      vals, out, ctl, bt, heads / kv_heads, hs, kv_dim, ctx_pad, qx, xs, xsum);
        return;
    }
    if (ctx <= kVrMaxCtx && hs % 32 == 0 && kv_dim % 4 == 0 && (reinterpret_cast<uintptr_t>(vals) & 15) == 0) {
        const int nsl = hs / kValSlice;
        RK_LAUNCH(att_values_reg_kernel, dim3(heads * nsl, ctl ? 1 : bt.tokens), dim3(kVrThreads),
                  att_values_reg_lds(ctx), s, att, att_stride, vals, out, ctl, bt, heads / kv_heads, hs, kv_dim, nsl,
                  (ctx + 3) & ~3, qx, xs, xsum);
        return;
    }
    if (vec)
        RK_LAUNCH((att_values_kernel<true, kValChunk>), grid, dim3(kValThreads), att_values_lds(ctx, kValChunk), s, att,
                  att_stride, vals, out, ctl, bt, heads / kv_heads, hs, kv_dim, ctx_pad, qx, xs, xsum);
    else
        RK_LAUNCH((att_values_kernel<false, kValChunk>), grid, dim3(kValThreads), att_values_lds(ctx, kValChunk), s, att,
                  att_stride, vals, out, ctl, bt, heads / kv_heads, hs, kv_dim, ctx_pad, qx, xs, xsum);
}

// ---------------------------------------------------------------------------
// The values and the Wo product in one launch.

struct AttWoArgs {
    const float *att, *vals;
    float *out;
    const int32_t *ctl;
    int32_t att_stride;
    int kv_mul, hs, kv_dim, nsl, ctx_pad;
    int8_t *qx;
    float *xs;
    int32_t *xsum;
    const uint8_t *w;  // Wo codes [rows][cols], scales [rows][cols/32]
    const float *ws;
    float *x;  // the residual: x[r] += the product's row r
    int rows, cols;
    unsigned long long *sync;
    int na, nw;  // values workgroups (producers), Wo workgroups
    QknIn qk;    // the QKN form's raw rows
};

// Wo rows a wave. With the register-held values (contexts past 256; about
// 200 VGPRs a lane, so a CU takes one workgroup of the launch) a Wo
// workgroup of 8 waves takes 32 rows: 4096 / 32 = 128 of them beside the
// 128 values workgroups of a 32-head model, one launch round on 256 CUs.
// With the short-context values (4 waves) it takes 16.
constexpr int kWoRowsPerWave = 4;

// Floats of one row's term buffer: [running sum L][block / 8], the row's
// C·32 blocks over 8 sums rounded up to 4 and padded by 4 (the writing
// lanes of a chunk in distinct banks).
constexpr int wo_k8p(int c) { return ((c * 32 / 8 + 3) & ~3) + 4; }

// Workgroup wi of the Wo product (C chunks of 1 KiB a row, K rows a wave):
// each wave requests all of its rows' codes and scales at once, then the
// workgroup waits for the values' Q8_0 output, reads it (agent-scope loads)
// and forms each row as MatVecQ8 does (internal/num/quant.go:158-180): the
// block terms float32(sum_b)·float32(ws_b·xs_b) into LDS by running sum
// b mod 8, eight lanes a row adding their sum's terms in block order, the
// sums combined ((0+1)+(2+3))+((4+5)+(6+7)) (DPP; addition commutes), then
// the residual add x[r] = x[r] + row (model.go:596, not canonicalised).
template <int C, int K, int W>
__device__ __forceinline__ void wo_after_values(const AttWoArgs &a, int wi) {
    extern __shared__ __align__(16) float smem[];
    constexpr int NS = K * C;
    constexpr int k8p = wo_k8p(C), rs = 8 * k8p;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int cols = a.cols, nb = cols >> 5, rows = a.rows;
    const int R0 = wi * (W * K) + wave * K;  // the wave's first row
    float *tbw = smem + wave * K * rs;
    const int g = lane >> 3, L = lane & 7, gk = g < K ? g : K - 1;
    const float ep0 = a.x[min(R0 + gk, rows - 1)];
    __amdgpu_buffer_rsrc_t rw[K], rsc[K];
#pragma unroll
    for (int h = 0; h < K; h++) {
        const int64_t r = min(R0 + h, rows - 1);
        rw[h] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(a.w + r * cols), 0, cols, kRsrcWord3);
        rsc[h] = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.ws + r * nb), 0, nb * 4, kRsrcWord3);
    }
    // lane offsets: 16 code bytes and their block's scale; the last chunk's
    // clamped into the row (lanes past it re-read its last piece, whose
    // blocks are never summed)
    const int wo = lane * 16, so = (lane >> 1) * 4;
    const int wl = min((C - 1) * 1024 + wo, cols - 16), sl = min((C - 1) * 128 + so, nb * 4 - 4);
    int4 wb[NS];
    float sb[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int h = s / C, c = s % C;
        const bool last = c == C - 1;
        const rk_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rw[h], last ? wl : wo, last ? 0 : c * 1024, kAuxStream);
        wb[s] = make_int4(v.x, v.y, v.z, v.w);
        sb[s] = __builtin_bit_cast(float,
                                   __builtin_amdgcn_raw_buffer_load_b32(rsc[h], last ? sl : so, last ? 0 : c * 128, 0));
        __builtin_amdgcn_sched_barrier(0);
    }

    sync_wait_ready(a.sync, a.nw, a.sync + kSyncError);

    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(a.qx, 0, cols, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(a.xs, 0, nb * 4, kRsrcWord3);
    int4 xq[C];
    float xsr[C];
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int o = c == C - 1 ? wl : c * 1024 + wo;
        const rk_v4i v = __builtin_amdgcn_raw_buffer_load_b128(rq, o, 0, kAuxCoherent);
        xq[c] = make_int4(v.x, v.y, v.z, v.w);
        xsr[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, (o >> 5) * 4, 0, kAuxCoherent));
    }
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int h = s / C, c = s % C;
        const int sm = pair_sum(dot16(wb[s], xq[c], 0));
        const float t = (float)sm * (sb[s] * xsr[c]);
        const int b = c * 32 + (lane >> 1);
        if ((lane & 1) == 0 && (c < C - 1 || b < nb)) tbw[h * rs + (b & 7) * k8p + (b >> 3)] = t;
    }
    float sum = 0.0f;
    {
        const float *p = tbw + gk * rs + L * k8p;
        if (nb == 128) {
            // (uniform: 4096 columns, sixteen terms a lane, read at once)
            const float4 *p4 = reinterpret_cast<const float4 *>(p);
            const float4 v0 = p4[0], v1 = p4[1], v2 = p4[2], v3 = p4[3];
            sum += v0.x;
            sum += v0.y;
            sum += v0.z;
            sum += v0.w;
            sum += v1.x;
            sum += v1.y;
            sum += v1.z;
            sum += v1.w;
            sum += v2.x;
            sum += v2.y;
            sum += v2.z;
            sum += v2.w;
            sum += v3.x;
            sum += v3.y;
            sum += v3.z;
            sum += v3.w;
        } else {
            const int cnt = L < nb ? (nb - L + 7) >> 3 : 0;
            int k = 0;
            for (; k + 4 <= cnt; k += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(p + k);
                sum += v.x;
                sum += v.y;
                sum += v.z;
                sum += v.w;
            }
            for (; k < cnt; k++) sum += p[k];
        }
    }
    sum = sum + dppf_x1(sum);
    sum = sum + dppf_x2(sum);
    sum = sum + __int_as_float(dpp_mirror8(__float_as_int(sum)));
    const int l = R0 + g;
    if (g < K && l < rows && L == 0) a.x[l] = ep0 + sum;
}

// Workgroups 0 .. na-1: the values (the producers: workgroup b the
// slice b mod nsl of head b / nsl, its Q8_0 block b); na .. na+nw-1: the Wo
// rows (waiting). The values workgroups come first in the grid, so they
// are dispatched first: a waiting workgroup never holds a place a producer
// still needs. SHORT: contexts up to 256 (att_values_kernel's work, 4
// waves), else att_values_reg_kernel's (8 waves).
// QKN: the short form with the scores formed in the values workgroups
// (att_values_body's QKN).
template <int C, bool SHORT, bool QKN = false>
__global__ __launch_bounds__(SHORT ? kValThreads : kVrThreads) void att_values_wo_kernel(AttWoArgs a) {
    static_assert(!QKN || SHORT, "QKN: the short form");
    if ((int)blockIdx.x < a.na) {
        if (SHORT)
            att_values_body<true, kValShortChunk, true, QKN>(a.att, a.att_stride, a.vals, a.out, a.ctl, AttBatch{},
                                                             a.kv_mul, a.hs, a.kv_dim, a.ctx_pad, a.qx, a.xs, a.xsum,
                                                             blockIdx.x / a.nsl, blockIdx.x % a.nsl, 0, a.sync, a.na,
                                                             &a.qk);
        else
            att_values_reg_body<true>(a.att, a.att_stride, a.vals, a.out, a.ctl, AttBatch{}, a.kv_mul, a.hs,
                                      a.kv_dim, a.nsl, a.ctx_pad, a.qx, a.xs, a.xsum, blockIdx.x, 0, a.sync, a.na);
        return;
    }
    wo_after_values<C, kWoRowsPerWave, (SHORT ? kValThreads : kVrThreads) / 64>(a, blockIdx.x - a.na);
}

bool launch_att_values_wo(const float *att, int32_t att_stride, const float *vals, float *out, const int32_t *ctl,
                          int ctx, int heads, int kv_heads, int hs, int kv_dim, int8_t *qx, float *xs, int32_t *xsum,
                          const uint8_t *wo_w, const float *wo_ws, int64_t wo_rows, int64_t wo_cols, float *x,
                          unsigned long long *sync, hipStream_t s, const QknIn *qk) {
    const bool shrt = ctx <= kValShortCtx;
    if (qk && (!shrt || hs != 128 || kv_dim != kv_heads * hs)) return false;
    const int wo_rows_wg = kWoRowsPerWave * (shrt ? kValThreads : kVrThreads) / 64;
    if (!ctl || !qx || !sync || ctx > kVrMaxCtx || hs % 32 != 0 || kv_dim % 4 != 0 ||
        (!shrt && (reinterpret_cast<uintptr_t>(vals) & 15) != 0))
        return false;
    if (wo_cols != (int64_t)heads * hs || wo_cols <= 3072 || wo_cols > 4096 || wo_rows <= 0 || wo_rows % wo_rows_wg)
        return false;
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute((const void *)att_values_wo_kernel<4, false>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)att_values_reg_lds(kVrMaxCtx));
    });
    AttWoArgs a{};
    a.att = att;
    a.vals = vals;
    a.out = out;
    a.ctl = ctl;
    a.att_stride = att_stride;
    a.kv_mul = heads / kv_heads;
    a.hs = hs;
    a.kv_dim = kv_dim;
    a.nsl = hs / kValSlice;
    a.ctx_pad = (ctx + 3) & ~3;
    a.qx = qx;
    a.xs = xs;
    a.xsum = xsum;
    a.w = wo_w;
    a.ws = wo_ws;
    a.x = x;
    a.rows = (int)wo_rows;
    a.cols = (int)wo_cols;
    a.sync = sync;
    a.na = heads * a.nsl;
    a.nw = (int)(wo_rows / wo_rows_wg);
    const size_t wo_lds = (size_t)wo_rows_wg * 8 * wo_k8p(4) * 4;
    if (shrt) {
        const int ctx_pad = (ctx + 3) & ~3;
        const size_t lds = ctx <= kValShortChunk ? (size_t)(ctx_pad + kValSlice * val_pitch(kValShortChunk)) * 4
                                                 : att_values_lds(ctx, kValShortChunk);
        if (qk) {
            a.qk = *qk;
            RK_LAUNCH((att_values_wo_kernel<4, true, true>), dim3((unsigned)(a.na + a.nw)), dim3(kValThreads),
                      std::max(lds, wo_lds), s, a);
        } else {
            RK_LAUNCH((att_values_wo_kernel<4, true>), dim3((unsigned)(a.na + a.nw)), dim3(kValThreads),
                      std::max(lds, wo_lds), s, a);
        }
    } else {
        RK_LAUNCH((att_values_wo_kernel<4, false>), dim3((unsigned)(a.na + a.nw)), dim3(kVrThreads),
                  std::max(att_values_reg_lds(ctx), wo_lds), s, a);
    }
    return true;
}

// QK-norm (internal/llm/model.go:551-558) and RoPE (:563-572) of one head
// per workgroup: q heads in place, k heads into the key cache (and their v
// heads into the value cache) at the position.
__global__ __launch_bounds__(64) void qknorm_rope_kernel(float *q, const float *k, const float *v,
                                                         const float *q_norm, const float *k_norm, float recip_hs,
                                                         float eps, const float *cos_t, const float *sin_t,
                                                         const int32_t *ctl, int32_t pos0, const int32_t *seq_pos,
                                                         int64_t cache_stride, float *kcache, float *vcache,
                                                         int heads, int hs, int kv_dim) {
    // a batch: token blockIdx.y at pos0 + blockIdx.y (or, independent
    // sequences, at seq_pos[blockIdx.y] in its own caches), rows
    // [tokens][heads·hs] and [tokens][kv_dim]
    const int z = blockIdx.y;
    const int pos = ctl ? ctl[kCtlPos] : seq_pos ? seq_pos[z] : pos0 + z;
    kcache += (int64_t)z * cache_stride;
    vcache += (int64_t)z * cache_stride;
    q += (int64_t)z * heads * hs;
    k += (int64_t)z * kv_dim;
    v += (int64_t)z * kv_dim;
    const int lane = threadIdx.x;
    const bool isq = (int)blockIdx.x < heads;
    const int head = isq ? blockIdx.x : blockIdx.x - heads;
    const float *x = isq ? q + (int64_t)head * hs : k + (int64_t)head * hs;
    float *dst = isq ? q + (int64_t)head * hs : kcache + (int64_t)pos * kv_dim + (int64_t)head * hs;
    qk_norm_rope_wave(x, isq ? q_norm : k_norm, recip_hs, eps, cos_t, sin_t, pos, hs, dst);
    if (!isq) {
        float *vd = vcache + (int64_t)pos * kv_dim + (int64_t)head * hs;
        const float *vs = v + (int64_t)head * hs;
        for (int i = lane; i < hs; i += 64) vd[i] = vs[i];
    }
}

void launch_qknorm_rope(float *q, const float *k, const float *v, const float *q_norm, const float *k_norm,
                        float recip_hs, float eps, const float *cos_t, const float *sin_t, const int32_t *ctl,
                        int32_t pos0, int tokens, float *kcache, float *vcache, int heads, int kv_heads, int hs,
                        hipStream_t s, const int32_t *seq_pos, int64_t cache_stride) {
    RK_LAUNCH(qknorm_rope_kernel, dim3(heads + kv_heads, ctl ? 1 : tokens), dim3(64), 0, s, q, k, v,
              q_norm, k_norm, recip_hs, eps, cos_t, sin_t, ctl, pos0, seq_pos, cache_stride, kcache, vcache, heads,
              hs, kv_heads * hs);
}

// Embedding row of the token at the position (internal/llm/model.go:216-231
// Row, :660-664 Embed): x_i = float32(q_i·scale_i/32); then RMSNorm(x) with
// the first layer's weights, quantized for its QKV product. One workgroup;
// every load is issued before the first use.
constexpr int kNormThreads = 1024;

constexpr int kNormGroups = (kMaxNormCols / 4 + kNormThreads - 1) / kNormThreads;

__global__ __launch_bounds__(kNormThreads) void embed_norm_kernel(const uint8_t *w, const float *scales, int q4,
                                                                  const int32_t *tokens, const int32_t *ctl, int dim,
                                                                  float *x, const float *norm_w, float recip_n,
                                                                  float eps, int8_t *qx, float *xs, int32_t *xsum) {
    extern __shared__ __align__(16) float sxe[];
    __shared__ float bcast;
    const int64_t tok = tokens[ctl[kCtlPos]];
    const int nb = dim >> 5, ng = dim >> 2;
    uint32_t cw[kNormGroups];
    float sc[kNormGroups];
    float4 wv[kNormGroups], xv[kNormGroups];
#pragma unroll
    for (int k = 0; k < kNormGroups; k++) {
        const int g = min((int)threadIdx.x + k * kNormThreads, ng - 1);  // elements 4g..4g+3
        const int i = 4 * g;
        // four codes: Q8 bytes 4g..; Q4 bytes of block i/32 holding j..j+3 (j = i mod 32)
        const uint8_t *cp = q4 ? w + tok * (dim / 2) + (i >> 5) * 16 + (i & 15) : w + tok * dim + i;
        cw[k] = *reinterpret_cast<const uint32_t *>(cp);
        sc[k] = scales[tok * nb + (i >> 5)];
        wv[k] = reinterpret_cast<const float4 *>(norm_w)[g];
    }
#pragma unroll
    for (int k = 0; k < kNormGroups; k++) {
        const int g = threadIdx.x + k * kNormThreads;
        int c[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int b = (int)((cw[k] >> (8 * e)) & 255u);
            c[e] = !q4 ? (int)(int8_t)b : ((((4 * g) & 31) < 16 ? (b & 15) : (b >> 4)) - 8);
        }
        xv[k] = make_float4((float)c[0] * sc[k], (float)c[1] * sc[k], (float)c[2] * sc[k], (float)c[3] * sc[k]);
        if (g < ng) reinterpret_cast<float4 *>(x)[g] = xv[k];
    }
    wg_norm_quant<kNormThreads, kNormGroups>(xv, wv, dim, recip_n, eps, qx, xs, xsum, sxe, &bcast);
}

void launch_embed_norm(const uint8_t *w, const float *scales, bool q4, const int32_t *tokens, const int32_t *ctl,
                       int dim, float *x, const float *norm_w, float recip_n, float eps, int8_t *qx, float *xs,
                       int32_t *xsum, hipStream_t s) {
    RK_LAUNCH(embed_norm_kernel, dim3(1), dim3(kNormThreads), norm_lds(dim), s, w, scales, q4 ? 1 : 0, tokens, ctl,
              dim, x, norm_w, recip_n, eps, qx, xs, xsum);
}

// Embedding rows of tokens[pos0..pos0+n) into x [n][dim] (the values
// embed_norm_kernel gives one position): workgroup per row, four elements a
// thread.
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint8_t *w, const float *scales, int q4,
                                                         const int32_t *tokens, int32_t pos0, int dim, float *x,
                                                         int64_t tok_stride, const int32_t *seq_pos) {
    // row z: tokens[pos0 + z], or (independent sequences) sequence z's token
    // at its position, tokens[z·tok_stride + seq_pos[z]]
    const int z = blockIdx.x;
    const int64_t tok = seq_pos ? tokens[(int64_t)z * tok_stride + seq_pos[z]] : tokens[pos0 + z];
    const int nb = dim >> 5, ng = dim >> 2;
    float *xr = x + (int64_t)blockIdx.x * dim;
    for (int g = threadIdx.x; g < ng; g += 256) {
        const int i = 4 * g;
        const uint8_t *cp = q4 ? w + tok * (dim / 2) + (i >> 5) * 16 + (i & 15) : w + tok * dim + i;
        const uint32_t cw = *reinterpret_cast<const uint32_t *>(cp);
        const float sc = scales[tok * nb + (i >> 5)];
        int c[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int b = (int)((cw >> (8 * e)) & 255u);
            c[e] = !q4 ? (int)(int8_t)b : (((i & 31) < 16 ? (b & 15) : (b >> 4)) - 8);
        }
        reinterpret_cast<float4 *>(xr)[g] =
            make_float4((float)c[0] * sc, (float)c[1] * sc, (float)c[2] * sc, (float)c[3] * sc);
    }
}

void launch_embed_rows(const uint8_t *w, const float *scales, bool q4, const int32_t *tokens, int32_t pos0, int n,
                       int dim, float *x, hipStream_t s, int64_t tok_stride, const int32_t *seq_pos) {
    RK_LAUNCH(embed_rows_kernel, dim3(n), dim3(256), 0, s, w, scales, q4 ? 1 : 0, tokens, pos0, dim, x, tok_stride,
              seq_pos);
}

__global__ __launch_bounds__(kNormThreads) void norm_quant_kernel(const float *x, int n, const float *norm_w,
                                                                  float recip_n, float eps, int8_t *qx, float *xs,
                                                                  int32_t *xsum) {
    extern __shared__ __align__(16) float sxn[];
    __shared__ float bcast;
    // a batch: vector blockIdx.x of [tokens][n]
    x += (int64_t)blockIdx.x * n;
    qx += (int64_t)blockIdx.x * n;
    xs += (int64_t)blockIdx.x * (n >> 5);
    xsum += (int64_t)blockIdx.x * (n >> 5);
    const int ng = n >> 2;
    float4 xv[kNormGroups], wv[kNormGroups];
#pragma unroll
    for (int k = 0; k < kNormGroups; k++) {
        const int g = min((int)threadIdx.x + k * kNormThreads, ng - 1);
        xv[k] = reinterpret_cast<const float4 *>(x)[g];
        wv[k] = reinterpret_cast<const float4 *>(norm_w)[g];
    }
    wg_norm_quant<kNormThreads, kNormGroups>(xv, wv, n, recip_n, eps, qx, xs, xsum, sxn, &bcast);
}

void launch_norm_quant(const float *x, int n, const float *norm_w, float recip_n, float eps, int8_t *qx, float *xs,
                       int32_t *xsum, hipStream_t s, int tokens) {
    RK_LAUNCH(norm_quant_kernel, dim3(tokens), dim3(kNormThreads), norm_lds(n), s, x, n, norm_w, recip_n, eps, qx, xs,
              xsum);
}

__global__ __launch_bounds__(64) void advance_kernel(int32_t *ctl, unsigned long long *amax, int32_t *tokens,
                                                     int32_t tokens_len) {
    const int lane = threadIdx.x;
    unsigned long long k = lane < kArgmaxSlots ? amax[lane] : 0ull;
    for (int w = 1; w < 64; w <<= 1) {
        const unsigned long long o = __shfl_xor(k, w);
        k = o > k ? o : k;
    }
    if (lane < kArgmaxSlots) amax[lane] = 0ull;
    if (lane == 0) {
        const int pos = ctl[kCtlPos];
        // no key: every logit NaN, and the first index stays (sample.go:46)
        if (pos + 1 >= ctl[kCtlPrompt] && pos + 1 < tokens_len)
            tokens[pos + 1] = k ? (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull)) : 0;
        ctl[kCtlPos] = pos + 1;
    }
}

void launch_advance(int32_t *ctl, unsigned long long *amax, int32_t *tokens, int32_t tokens_len, hipStream_t s) {
    RK_LAUNCH(advance_kernel, dim3(1), dim3(64), 0, s, ctl, amax, tokens, tokens_len);
}

}  // namespace rk
