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
// the workgroup itself into LDS before the stream starts (kProQuant,
// kProNorm): the input's loads are issued first, then the first weight
// chunks, so the prologue runs while those weights are on their way.
#include "rk_dev.h"
#include "rk_fused.h"

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
    __shared__ float s_bcast;
    __shared__ float s_wv[W];
    __shared__ int s_wi[W];
    __shared__ int s_last;
    constexpr bool PAIR = (EPI == kEpQKV || EPI == kEpSilu);
    constexpr int NT = 64 * W;
    constexpr int MAXG = PRO == kProGlobal ? 1 : (kMaxLdsCols / 4 + NT - 1) / NT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cols = a.cols, nb = cols >> 5;
    const int rowbytes = FMT == kFmtQ8 ? cols : cols >> 1;
    const int C = FMT == kFmtQ8 ? (cols + 1023) >> 10 : (nb + 63) >> 6;

    int pos = 0;
    bool work = true;
    if (EPI == kEpQKV || EPI == kEpLogits) pos = a.ctl[kCtlPos];
    if (EPI == kEpLogits && a.gate && pos + 1 < a.ctl[kCtlPrompt]) work = false;

    const int R0 = blockIdx.x * a.rows_per_wg;
    const int R1 = min(a.rows, R0 + a.rows_per_wg);
    const int n = R1 - R0;
    int nrows = 0;
    if (work) {
        if (PAIR) {
            const int np = (n + 1) >> 1;
            if (wave < np) {
                nrows = 2 * ((np - 1 - wave) / W + 1);
                if ((n & 1) && (np - 1 - wave) % W == 0) nrows -= 1;
            }
        } else {
            nrows = wave < n ? (n - 1 - wave) / W + 1 : 0;
        }
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

    // ---- input loads (LDS prologues): issued before any weight ----
    float4 xv[MAXG];
    float4 nw[PRO == kProNorm ? MAXG : 1];
    if (PRO != kProGlobal && work) {
#pragma unroll
        for (int k = 0; k < MAXG; k++) {
            const int g = threadIdx.x + k * NT;
            xv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (g < (cols >> 2)) xv[k] = reinterpret_cast<const float4 *>(a.x)[g];
            if (PRO == kProNorm) {
                nw[k] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (g < (cols >> 2)) nw[k] = reinterpret_cast<const float4 *>(a.norm_w)[g];
            }
        }
    }

    // ---- weight stream: U chunks in flight ----
    int lp = wave, lh = 0, lc = 0;
    RowSrc ls = row_src<EPI>(a, row_of(lp, lh), rowbytes, nb);
    int4 wb[U], xb0[U], xb1[U];
    float sb[U], xsb[U];
    int xsumb[U];
    auto load = [&](int j) {
        wb[j] = make_int4(0, 0, 0, 0);
        sb[j] = 0.0f;
        if (PRO == kProGlobal) {
            xb0[j] = xb1[j] = make_int4(0, 0, 0, 0);
            xsb[j] = 0.0f;
            xsumb[j] = 0;
        }
        if (FMT == kFmtQ8) {
            const int off = lc * 1024 + lane * 16;
            if (off < cols) {
                wb[j] = load_stream16(ls.w + off);
                sb[j] = ls.ws[off >> 5];
                if (PRO == kProGlobal) {
                    xb0[j] = *reinterpret_cast<const int4 *>(a.qx + off);
                    xsb[j] = a.xs[off >> 5];
                }
            }
        } else {
            const int blk = lc * 64 + lane;
            if (blk < nb) {
                wb[j] = load_stream16(ls.w + blk * 16);
                sb[j] = ls.ws[blk];
                if (PRO == kProGlobal) {
                    xb0[j] = *reinterpret_cast<const int4 *>(a.qx + blk * 32);
                    xb1[j] = *reinterpret_cast<const int4 *>(a.qx + blk * 32 + 16);
                    xsb[j] = a.xs[blk];
                    xsumb[j] = a.xsum[blk];
                }
            }
        }
        if (++lc == C) {
            lc = 0;
            next_row(lp, lh);
            ls = row_src<EPI>(a, row_of(lp, lh), rowbytes, nb);
        }
    };
#pragma unroll
    for (int j = 0; j < U; j++)
        if (j < nsteps) load(j);

    // ---- prologue: RMSNorm (internal/llm/model.go:632-638) and Q8_0
    // quantization (internal/num/quant.go:34-53) of the input, into LDS ----
    int8_t *sqx = reinterpret_cast<int8_t *>(lds);
    float *sxs = reinterpret_cast<float *>(lds + a.lds_xs);
    int *sxsum = reinterpret_cast<int *>(lds + a.lds_xsum);
    if (PRO != kProGlobal && work) {
        if (PRO == kProNorm) {
            float *sx = reinterpret_cast<float *>(lds + a.lds_x);
#pragma unroll
            for (int k = 0; k < MAXG; k++) {
                const int g = threadIdx.x + k * NT;
                if (g < (cols >> 2)) reinterpret_cast<float4 *>(sx)[g] = xv[k];
            }
            __syncthreads();
            if (wave == 0) {
                float s = 0.0f;
                if (lane < 32)
                    for (int i = lane; i < cols; i += 32) s += sx[i] * sx[i];
                const float dot = dot32_reduce(s);
                if (lane == 0) s_bcast = rsqrt32((dot * a.recip_n) + a.eps);
            }
            __syncthreads();
            const float r = s_bcast;
#pragma unroll
            for (int k = 0; k < MAXG; k++) {
                xv[k].x = nw[k].x * (r * xv[k].x);
                xv[k].y = nw[k].y * (r * xv[k].y);
                xv[k].z = nw[k].z * (r * xv[k].z);
                xv[k].w = nw[k].w * (r * xv[k].w);
            }
        }
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
        __syncthreads();
    }

    // ---- stream and reduce ----
    float acc = 0.0f, held = 0.0f;
    float best_v = 0.0f;
    int best_i = -1;
    int pp = wave, ph = 0, pc = 0;
    const int half = a.hs >> 1;
    auto epilogue = [&](int l, float res) {
        if (EPI == kEpSilu) {
            if ((l & 1) == 0)
                held = res;
            else
                a.seg[0].out[l >> 1] = silu_mul(held, res);
            return;
        }
        if (EPI == kEpQKV) {
            const int lg = a.row_base + l;
            float v = res;
            if (a.bias) v = v + a.bias[lg];
            if ((l & 1) == 0) {
                held = v;
                return;
            }
            const float v0 = held, v1 = v;
            const int i0 = lg - 1;
            if (i0 < a.qdim + a.kvdim) {
                const bool isq = i0 < a.qdim;
                const int i = isq ? i0 : i0 - a.qdim;
                const int pi = (i % a.hs) >> 1;
                const float co = a.cos_t[(int64_t)pos * half + pi], si = a.sin_t[(int64_t)pos * half + pi];
                const float r0 = (v0 * co) - (v1 * si);
                const float r1 = (v0 * si) + (v1 * co);
                float *dst = isq ? a.seg[0].out + i : a.kcache + (int64_t)pos * a.kvdim + i;
                dst[0] = r0;
                dst[1] = r1;
            } else {
                float *dst = a.vcache + (int64_t)pos * a.kvdim + (i0 - a.qdim - a.kvdim);
                dst[0] = v0;
                dst[1] = v1;
            }
            return;
        }
        const RowSrc rs = row_src<EPI>(a, l, rowbytes, nb);
        float *o = rs.out + rs.r;
        if (EPI == kEpStore) {
            *o = a.bias ? res + a.bias[l] : res;
        } else if (EPI == kEpAdd) {
            *o = *o + res;
        } else if (EPI == kEpAddCanon) {
            *o = canonical(*o + res);
        } else if (EPI == kEpLogits) {
            *o = res;
            if (res == res) argmax_merge(best_v, best_i, res, rs.r);
        }
    };

    auto process = [&](int j) {
        float t;
        if (FMT == kFmtQ8) {
            int4 xq = xb0[j];
            float xsv = xsb[j];
            if (PRO != kProGlobal) {
                const int off = pc * 1024 + lane * 16;
                xq = make_int4(0, 0, 0, 0);
                xsv = 0.0f;
                if (off < cols) {
                    xq = *reinterpret_cast<const int4 *>(sqx + off);
                    xsv = sxs[off >> 5];
                }
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
                const int blk = pc * 64 + lane;
                x0 = x1 = make_int4(0, 0, 0, 0);
                xsv = 0.0f;
                xsum = 0;
                if (blk < nb) {
                    x0 = *reinterpret_cast<const int4 *>(sqx + blk * 32);
                    x1 = *reinterpret_cast<const int4 *>(sqx + blk * 32 + 16);
                    xsv = sxs[blk];
                    xsum = sxsum[blk];
                }
            }
            const int4 w = wb[j];
            const int4 lo = make_int4(w.x & 0x0F0F0F0F, w.y & 0x0F0F0F0F, w.z & 0x0F0F0F0F, w.w & 0x0F0F0F0F);
            const int4 hi = make_int4((int)(((uint32_t)w.x >> 4) & 0x0F0F0F0Fu), (int)(((uint32_t)w.y >> 4) & 0x0F0F0F0Fu),
                                      (int)(((uint32_t)w.z >> 4) & 0x0F0F0F0Fu), (int)(((uint32_t)w.w >> 4) & 0x0F0F0F0Fu));
            // nibble j is w_j + 8: sum_b = Σ lo·x_j + Σ hi·x_j+16 - 8·Σ x
            const int s = dot16(hi, x1, dot16(lo, x0, 0)) - 8 * xsum;
            t = (float)s * (sb[j] * xsv);
            // block 64pc+l is in lane l; running sum L (lane L) takes lanes
            // L, L+8, ..., L+56.
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
            if (st + j < nsteps) {
                process(j);
                if (st + j + U < nsteps) load(j);
            }
        }
    }

    if (EPI == kEpLogits) {
        // Greedy argmax over all rows: per wave, per workgroup, then the last
        // workgroup to finish merges the partials, stores the next token and
        // advances the position (all other workgroups read it already).
        if (lane == 0) {
            s_wv[wave] = best_v;
            s_wi[wave] = best_i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float bv = 0.0f;
            int bi = -1;
            for (int w = 0; w < W; w++) argmax_merge(bv, bi, s_wv[w], s_wi[w]);
            a.part_v[blockIdx.x] = bv;
            a.part_i[blockIdx.x] = bi;
            __threadfence();
            s_last = atomicAdd(&a.ctl[kCtlDone], 1) == (int)gridDim.x - 1;
        }
        __syncthreads();
        if (s_last) {
            __threadfence();
            float bv = 0.0f;
            int bi = -1;
            for (int i = threadIdx.x; i < (int)gridDim.x; i += NT) argmax_merge(bv, bi, a.part_v[i], a.part_i[i]);
            // the merge is a maximum under a total order: any fold order
            for (int w = 1; w < 64; w <<= 1) {
                const float ov = __shfl_xor(bv, w);
                const int oi = __shfl_xor(bi, w);
                argmax_merge(bv, bi, ov, oi);
            }
            if (lane == 0) {
                s_wv[wave] = bv;
                s_wi[wave] = bi;
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                float fv = 0.0f;
                int fi = -1;
                for (int w = 0; w < W; w++) argmax_merge(fv, fi, s_wv[w], s_wi[w]);
                if (work && pos + 1 < a.tokens_len) {
                    const float l0 = a.seg[0].out[0];
                    a.tokens[pos + 1] = (fi < 0 || l0 != l0) ? 0 : fi;
                }
                a.ctl[kCtlPos] = pos + 1;
                a.ctl[kCtlDone] = 0;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Launch: the host sizes the grid (about two workgroups per CU, rows split
// evenly, pairs kept whole) and the LDS layout.

template <int FMT, int PRO, int EPI, int W>
static void launch_one(const FusedArgs &a, unsigned grid, size_t lds, hipStream_t s) {
    RK_LAUNCH((fused_kernel<FMT, PRO, EPI, W, 2>), dim3(grid), dim3(64 * W), lds, s, a);
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

static void lds_layout(FusedArgs &a, int pro) {
    const int cols = a.cols, nb = cols >> 5;
    a.lds_xs = align16(cols);
    a.lds_xsum = a.lds_xs + align16(nb * 4);
    a.lds_x = a.lds_xsum + align16(nb * 4);
    a.lds_bytes = a.lds_x + (pro == kProNorm ? cols * 4 : 0);
}

bool fused_fits(int pro, int cols) {
    if (pro == kProGlobal) return true;
    if (cols > kMaxLdsCols || cols % 32 != 0) return false;
    FusedArgs a{};
    a.cols = cols;
    lds_layout(a, pro);
    return a.lds_bytes <= kMaxDynLds;
}

bool launch_fused(int fmt, int pro, int epi, FusedArgs a, int cu, hipStream_t s) {
    if (a.rows <= 0) return true;
    if (a.cols <= 0 || a.cols % 32 != 0 || !fused_fits(pro, a.cols)) return false;
    size_t lds = 0;
    if (pro != kProGlobal) {
        lds_layout(a, pro);
        lds = (size_t)a.lds_bytes;
    }
    const bool pair = epi == kEpQKV || epi == kEpSilu;
    const int64_t target = (int64_t)(cu > 0 ? cu : 256) * 2;
    int64_t rpw = (a.rows + target - 1) / target;
    if (pair) rpw = (rpw + 1) & ~1;
    if (epi == kEpLogits) {
        const int64_t min_rpw = (a.rows + kMaxArgmaxParts - 1) / kMaxArgmaxParts;
        if (rpw < min_rpw) rpw = min_rpw;
    }
    a.rows_per_wg = (int32_t)rpw;
    const unsigned grid = (unsigned)((a.rows + rpw - 1) / rpw);
    const int64_t units = pair ? (rpw + 1) / 2 : rpw;
    const bool wide = units >= 12;
    if (fmt == kFmtQ8)
        return wide ? launch_pro<kFmtQ8, 16>(pro, epi, a, grid, lds, s) : launch_pro<kFmtQ8, 8>(pro, epi, a, grid, lds, s);
    return wide ? launch_pro<kFmtQ4, 16>(pro, epi, a, grid, lds, s) : launch_pro<kFmtQ4, 8>(pro, epi, a, grid, lds, s);
}

// ---------------------------------------------------------------------------
// Attention of the position ctl[kCtlPos] (internal/llm/model.go:575-591).

constexpr int kScorePositions = 32;  // positions per workgroup

// score_t = float32(Dot32(q_h, k_t)·invSqrt), t <= position: a half-wave
// per position, grid (heads, position tiles); tiles past the position exit.
__global__ __launch_bounds__(256) void att_scores_kernel(const float *q, const float *keys, float *att,
                                                         int32_t att_stride, const int32_t *ctl, int kv_mul, int hs,
                                                         int kv_dim, float inv_sqrt) {
    const int T = ctl[kCtlPos] + 1;
    const int t0 = blockIdx.y * kScorePositions;
    if (t0 >= T) return;
    const int h = blockIdx.x, g = h / kv_mul;
    const int half = threadIdx.x >> 5, hl = threadIdx.x & 31;
    const float *qh = q + (int64_t)h * hs;
    for (int tt = half; tt < kScorePositions; tt += 8) {
        const int t = t0 + tt;
        const bool valid = t < T;
        const float *kt = keys + (int64_t)(valid ? t : 0) * kv_dim + (int64_t)g * hs;
        const float d = dot32_half(qh, kt, hs, hl, valid);
        if (valid && hl == 0) att[(int64_t)h * att_stride + t] = d * inv_sqrt;
    }
}

void launch_att_scores(const float *q, const float *keys, float *att, int32_t att_stride, const int32_t *ctl,
                       int ctx, int heads, int kv_heads, int hs, int kv_dim, float inv_sqrt, hipStream_t s) {
    const dim3 grid(heads, (ctx + kScorePositions - 1) / kScorePositions);
    RK_LAUNCH(att_scores_kernel, grid, dim3(256), 0, s, q, keys, att, att_stride, ctl, heads / kv_heads, hs, kv_dim,
              inv_sqrt);
}

// Softmax of a head's scores (Go max, Exp32, one sequential sum, ·Recip32)
// and the weighted values, out_i = Σ_t a_t·v_t,i in t order from +0. One
// wave per 64 elements of a head: grid (heads, ceil(hs/64)); each wave
// redoes its head's softmax (cheap) so no wave waits on another.
__global__ __launch_bounds__(64) void att_values_kernel(const float *att, int32_t att_stride, const float *vals,
                                                        float *out, const int32_t *ctl, int kv_mul, int hs,
                                                        int kv_dim) {
    extern __shared__ float sa[];  // [T] weights
    const int T = ctl[kCtlPos] + 1;
    const int h = blockIdx.x, g = h / kv_mul;
    const int lane = threadIdx.x;
    const float *ah = att + (int64_t)h * att_stride;
    float m = ah[0];
    for (int t = lane; t < T; t += 64) {
        const float v = ah[t];
        sa[t] = v;
        m = gomax(m, v);
    }
    for (int w = 1; w < 64; w <<= 1) m = gomax(m, __shfl_xor(m, w));
    for (int t = lane; t < T; t += 64) sa[t] = exp32(sa[t] - m);
    __syncthreads();
    if (lane == 0) {
        float sum = 0.0f;
        int t = 0;
        for (; t + 8 <= T; t += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = sa[t + j];
#pragma unroll
            for (int j = 0; j < 8; j++) sum += v[j];
        }
        for (; t < T; t++) sum += sa[t];
        sa[T] = recip32(sum);
    }
    __syncthreads();
    const float inv = sa[T];
    for (int t = lane; t < T; t += 64) sa[t] = sa[t] * inv;
    __syncthreads();
    const int i = blockIdx.y * 64 + lane;
    if (i >= hs) return;
    const float *v = vals + (int64_t)g * hs + i;
    float acc = 0.0f;
    int t = 0;
    for (; t + 8 <= T; t += 8) {
        float vv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) vv[j] = v[(int64_t)(t + j) * kv_dim];
#pragma unroll
        for (int j = 0; j < 8; j++) acc += sa[t + j] * vv[j];
    }
    for (; t < T; t++) acc += sa[t] * v[(int64_t)t * kv_dim];
    out[(int64_t)h * hs + i] = acc;
}

void launch_att_values(const float *att, int32_t att_stride, const float *vals, float *out, const int32_t *ctl,
                       int ctx, int heads, int kv_heads, int hs, int kv_dim, hipStream_t s) {
    const dim3 grid(heads, (hs + 63) / 64);
    RK_LAUNCH(att_values_kernel, grid, dim3(64), (size_t)(ctx + 1) * 4, s, att, att_stride, vals, out, ctl,
              heads / kv_heads, hs, kv_dim);
}

// QK-norm (internal/llm/model.go:551-558) and RoPE (:563-572) of one head
// per workgroup: q heads in place, k heads into the key cache (and their v
// heads into the value cache) at the position.
__global__ __launch_bounds__(64) void qknorm_rope_kernel(float *q, const float *k, const float *v,
                                                         const float *q_norm, const float *k_norm, float recip_hs,
                                                         float eps, const float *cos_t, const float *sin_t,
                                                         const int32_t *ctl, float *kcache, float *vcache, int heads,
                                                         int hs, int kv_dim) {
    extern __shared__ float sy[];  // [hs]
    const int pos = ctl[kCtlPos];
    const int lane = threadIdx.x;
    const bool isq = (int)blockIdx.x < heads;
    const int head = isq ? blockIdx.x : blockIdx.x - heads;
    const float *x = isq ? q + (int64_t)head * hs : k + (int64_t)head * hs;
    const float *w = isq ? q_norm : k_norm;
    const float dot = __shfl(dot32_half(x, x, hs, lane & 31, lane < 32), 0);
    const float r = rsqrt32((dot * recip_hs) + eps);
    for (int i = lane; i < hs; i += 64) sy[i] = w[i] * (r * x[i]);
    __syncthreads();
    const int half = hs >> 1;
    float *dst = isq ? q + (int64_t)head * hs : kcache + (int64_t)pos * kv_dim + (int64_t)head * hs;
    for (int p = lane; p < half; p += 64) {
        const float co = cos_t[(int64_t)pos * half + p], si = sin_t[(int64_t)pos * half + p];
        const float v0 = sy[2 * p], v1 = sy[2 * p + 1];
        dst[2 * p] = (v0 * co) - (v1 * si);
        dst[2 * p + 1] = (v0 * si) + (v1 * co);
    }
    if (!isq) {
        float *vd = vcache + (int64_t)pos * kv_dim + (int64_t)head * hs;
        const float *vs = v + (int64_t)head * hs;
        for (int i = lane; i < hs; i += 64) vd[i] = vs[i];
    }
}

void launch_qknorm_rope(float *q, const float *k, const float *v, const float *q_norm, const float *k_norm,
                        float recip_hs, float eps, const float *cos_t, const float *sin_t, const int32_t *ctl,
                        float *kcache, float *vcache, int heads, int kv_heads, int hs, hipStream_t s) {
    RK_LAUNCH(qknorm_rope_kernel, dim3(heads + kv_heads), dim3(64), (size_t)hs * 4, s, q, k, v, q_norm, k_norm,
              recip_hs, eps, cos_t, sin_t, ctl, kcache, vcache, heads, hs, kv_heads * hs);
}

// Embedding row of the token at the position (internal/llm/model.go:216-231
// Row, :660-664 Embed): x_i = float32(q_i·scale_i/32).
__global__ void embed_pos_kernel(const uint8_t *w, const float *scales, int q4, const int32_t *tokens,
                                 const int32_t *ctl, int dim, float *x) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    const int64_t tok = tokens[ctl[kCtlPos]];
    const int nb = dim >> 5;
    const float d = scales[tok * nb + (i >> 5)];
    if (!q4) {
        x[i] = (float)reinterpret_cast<const int8_t *>(w)[tok * dim + i] * d;
    } else {
        const uint8_t b = w[tok * (dim / 2) + (i >> 5) * 16 + (i & 15)];
        const int c = ((i & 31) < 16 ? (b & 15) : (b >> 4)) - 8;
        x[i] = (float)c * d;
    }
}

void launch_embed_pos(const uint8_t *w, const float *scales, bool q4, const int32_t *tokens, const int32_t *ctl,
                      int dim, float *x, hipStream_t s) {
    RK_LAUNCH(embed_pos_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, w, scales, q4 ? 1 : 0, tokens, ctl, dim, x);
}

}  // namespace rk
