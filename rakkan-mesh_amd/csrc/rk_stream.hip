// rk_stream.hip — the batch-1 quantized products with a static per-wave
// schedule, for gfx950: the fast path of launch_fused (rk_fused.hip), for
// the input widths instantiated below. Results are fused_kernel's, bit for
// bit: the Q8_0 input blocks (internal/num/quant.go:34-53), exact integer
// block sums, and per row the eight running sums of quant.go:158-164 in
// block order with their fixed tree ((0+1)+(2+3))+((4+5)+(6+7)).
//
// Work layout. A workgroup owns `nbatch` batches of W·K consecutive output
// rows; in a batch, wave w owns rows w·K .. w·K+K-1 whole. A row is C
// chunks (Q8: 1 KiB of codes, 16 bytes per lane; Q4: 64 blocks, one 16-byte
// block per lane), so a wave walks its K·C chunks in memory order with U in
// flight. The walk is unrolled at compile time: each chunk's load is issued
// once, after the chunk U steps earlier has been used, and none past the
// wave's last chunk (the last U chunks of a batch prefetch the next batch's
// first ones, when there is one). The waits are then fixed counts, and no
// load reads memory the product does not need.
//
// Each chunk leaves its per-block terms float32(sum_b)·float32(ws_b·xs_b) in
// LDS, laid out [running sum L = b mod 8][b / 8]. After a batch, eight lanes
// per row add their running sum's terms in block order from +0 and combine
// the eight sums by DPP (xor 1, xor 2, mirror), which is the reference tree
// since float addition commutes. The epilogues are fused_kernel's.
#include <algorithm>
#include <mutex>

#include "rk_dev.h"
#include "rk_fused.h"

namespace rk {

namespace {

struct Src {
    const uint8_t *w;
    const float *ws;
};

// Buffer resources of one row's codes and scales.
struct Row {
    __amdgpu_buffer_rsrc_t w, s;
};


// Codes and scales of logical row l: up to three matrices concatenated, or
// (kEpSilu) W1 and W3 interleaved row by row. l is wave-uniform, so this
// is scalar work.
template <int EPI>
__device__ __forceinline__ Src stream_src(const FusedArgs &a, int l, int rowbytes, int nb) {
    const uint8_t *w;
    const float *ws;
    int64_t r;
    if (EPI == kEpSilu) {
        r = l >> 1;
        w = (l & 1) ? a.seg[1].w : a.seg[0].w;
        ws = (l & 1) ? a.seg[1].ws : a.seg[0].ws;
    } else {
        r = l;
        w = a.seg[0].w;
        ws = a.seg[0].ws;
        if (a.nseg > 1 && r >= a.seg[0].rows) {
            r -= a.seg[0].rows;
            w = a.seg[1].w;
            ws = a.seg[1].ws;
            if (a.nseg > 2 && r >= a.seg[1].rows) {
                r -= a.seg[1].rows;
                w = a.seg[2].w;
                ws = a.seg[2].ws;
            }
        }
    }
    return Src{w + r * rowbytes, ws + r * nb};
}

// Output word of logical row l for the store, residual and logits
// epilogues (the segment's output at the row).
__device__ __forceinline__ float *stream_out(const FusedArgs &a, int l) {
    int64_t r = l;
    float *o = a.seg[0].out;
    if (a.nseg > 1 && r >= a.seg[0].rows) {
        r -= a.seg[0].rows;
        o = a.seg[1].out;
        if (a.nseg > 2 && r >= a.seg[1].rows) {
            r -= a.seg[1].rows;
            o = a.seg[2].out;
        }
    }
    return o + r;
}

// Smallest workgroup (waves) an instance takes: its prologue keeps the
// input's pieces per thread in registers (loaded before the weights, so a
// wait for them never waits for a weight chunk), a count fixed per instance.
constexpr int stream_wmin(int fmt, int pro, int c) {
    return pro == kProGlobal ? ((fmt == kFmtQ8 ? c <= 4 : c <= 2) ? 4 : 8)
                             : ((fmt == kFmtQ8 ? c * 256 : c * 512) > 1024 ? 12 : 8);
}

// RMSNorm (internal/llm/model.go:632-638: ss = Dot32(x,x)·recip_n + eps,
// out_i = w_i·(Rsqrt32(ss)·x_i)) of x and the Q8_0 quantization of the
// result (internal/num/quant.go:34-53) into qx/xs/xsum, by a workgroup of
// nt threads; thread t holds groups t + k·nt (four values each) of x and w.
// sx: LDS for x transposed (32 rows of `pitch` floats). Same steps and
// order as the stand-alone norm kernel.
template <int MG>
__device__ void norm_quant_rt(const float4 *xv, const float4 *wv, int n, int nt, float recip_n, float eps, int8_t *qx,
                              float *xs, int32_t *xsum, float *sx, float *bcast) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int ng = n >> 2;
    const int steps = n >> 5, pitch = ((steps + 3) & ~3) + 4;
#pragma unroll
    for (int k = 0; k < MG; k++) {
        const int g = tid + k * nt;
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
        float s = 0.0f;
        if (lane < 32) {  // Dot32 running sum `lane`: x_i·x_i, i = lane + 32m, m ascending
            const float *row = sx + lane * pitch;
            int m = 0;
            for (; m + 16 <= steps; m += 16) s = lds_sq_fixed<16>(row + m, s);
            for (; m < steps; m++) s += row[m] * row[m];
        }
        const float dot = dot32_reduce(s);
        if (lane == 0) *bcast = rsqrt32((dot * recip_n) + eps);
    }
    __syncthreads();
    const float r = *bcast;
#pragma unroll
    for (int k = 0; k < MG; k++) {
        if (k * nt < ng) {  // uniform
            const int g = tid + k * nt;
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

// LDS of the transposed x of norm_quant_rt for n values.
size_t stream_norm_lds(int n) { return (size_t)32 * ((((n >> 5) + 3) & ~3) + 4) * 4; }

// Floats per running sum in the term buffer for rows of C chunks: the
// widest row's blocks / 8, rounded up to a multiple of 4 and padded by 4 so
// the 32 writing lanes of a Q8 chunk fall in distinct banks.
constexpr int stream_k8p(int fmt, int c) { return (((fmt == kFmtQ8 ? c * 32 : c * 64) / 8 + 3) & ~3) + 4; }

// PF: the last U steps of a batch prefetch the next batch's first chunks.
// Without (a workgroup of one batch) those steps issue no loads, and the
// waits are fixed counts all the same.
template <int FMT, int PRO, int EPI, int K, int U, int C, bool PF>
__global__ __launch_bounds__(1024) void stream_kernel(FusedArgs a, int nbatch) {
    extern __shared__ __align__(16) char lds[];
    __shared__ float s_wv[16];
    __shared__ int s_wi[16];
    __shared__ float s_rn;
    constexpr bool Q8 = FMT == kFmtQ8;
    constexpr bool XR = Q8 ? C <= 4 : C <= 2;  // the input's chunks in registers
    constexpr int NS = K * C;
    static_assert(NS % U == 0, "a batch is a whole number of load rounds");
    constexpr int GPC = Q8 ? 256 : 512;  // groups of four input values per chunk
    constexpr int NTMIN = 64 * stream_wmin(FMT, PRO, C);
    constexpr int MG = PRO == kProNorm ? (C * GPC + NTMIN - 1) / NTMIN : 1;
    static_assert(PRO != kProQuant || (Q8 ? C * 32 : C * 64) <= NTMIN, "the quantize prologue takes one block per thread");
    constexpr int MQ = ((Q8 ? 64 : 128) * C + NTMIN - 1) / NTMIN;  // 16-byte pieces of qx per thread
    constexpr int MB = ((Q8 ? 32 : 64) * C + NTMIN - 1) / NTMIN;   // blocks per thread
    constexpr bool PAIR = EPI == kEpQKV || EPI == kEpSilu;
    static_assert(!PAIR || K % 2 == 0, "pair epilogues keep both rows of a pair in one wave");

    const int nt = blockDim.x, W = nt >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int cols = a.cols, nb = cols >> 5;
    const int rowbytes = Q8 ? cols : cols >> 1;
    const int RB = W * K;
    const int R0 = blockIdx.x * a.rows_per_wg;
    constexpr int k8p = stream_k8p(FMT, C), rs = 8 * k8p;

    int pos = 0;
    if (EPI == kEpQKV || EPI == kEpLogits) pos = a.ctl[kCtlPos];
    if (EPI == kEpLogits && a.gate && pos + 1 < a.ctl[kCtlPrompt]) return;  // uniform over the grid

    int8_t *sqx = reinterpret_cast<int8_t *>(lds);
    float *sxs = reinterpret_cast<float *>(lds + a.lds_xs);
    int *sxsum = reinterpret_cast<int *>(lds + a.lds_xsum);
    float *tbw = reinterpret_cast<float *>(lds + a.lds_res) + wave * K * rs;
    float *sh = reinterpret_cast<float *>(lds + a.lds_ep);  // kEpSilu: the workgroup's h

    // This lane's piece of each chunk: Q8 byte offset (also the input's),
    // Q4 block (clamped into the row; what lies past it is never summed).
    // (only the last chunk can reach past the row, so the others fold into
    // immediate offsets)
    auto oc = [&](int c) {
        return Q8 ? (c == C - 1 ? min(c * 1024 + lane * 16, cols - 16) : c * 1024 + lane * 16)
                  : (c == C - 1 ? min(c * 64 + lane, nb - 1) : c * 64 + lane);
    };

    // ---- (1) the input's loads ----
    float4 xv[PRO == kProNorm ? MG : 1], wv[PRO == kProNorm ? MG : 1];
    float4 xb[8];  // kProQuant: the thread's block of x (block threadIdx.x)
    int4 xq0[XR ? C : 1], xq1[(XR && !Q8) ? C : 1];
    float xsr[XR ? C : 1];
    int xsm[(XR && !Q8) ? C : 1];
    // (every thread loads its MG/MQ/MB pieces, clamped into the vector, so
    // the pieces stay in registers)
    if (PRO == kProNorm) {
        const int ng = cols >> 2;
#pragma unroll
        for (int k = 0; k < MG; k++) {
            const int g = min((int)threadIdx.x + k * nt, ng - 1);
            xv[k] = reinterpret_cast<const float4 *>(a.x)[g];
            wv[k] = reinterpret_cast<const float4 *>(a.norm_w)[g];
        }
    } else if (PRO == kProQuant && XR) {
        // only the waves that quantize a block load x
        if ((int)threadIdx.x - lane < nb) {  // uniform
            const float4 *xp = reinterpret_cast<const float4 *>(a.x) + 8 * min((int)threadIdx.x, nb - 1);
#pragma unroll
            for (int k = 0; k < 8; k++) xb[k] = xp[k];
        }
    } else if (PRO == kProQuant) {
        // A wide input (rows of more than 4 chunks): x staged in LDS as it
        // lies in memory (the term buffer's room, unused until the batches)
        // by direct-to-LDS loads of 1 KiB, wave w taking blocks
        // 64w .. 64w+63; then a barrier, so every wave's loads of x are
        // issued before any weight load of the workgroup (the vector memory
        // queue is in issue order: x behind the weights' first rounds came
        // in microseconds late).
        if (wave * 64 < nb) {  // uniform
            const int nq4 = cols >> 2;
            float *xf = reinterpret_cast<float *>(lds + a.lds_norm);
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int p0 = (wave * 64 + 8 * k) * 8;  // the load's first 16-byte piece
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const float4 *>(a.x) + min(p0 + lane, nq4 - 1),
                                                 lds_ptr(xf + 4 * p0), 16, 0, 0);
            }
        }
        asm volatile("s_barrier" ::: "memory");  // issue order only: no wait for the loads
    } else if (XR) {
#pragma unroll
        for (int c = 0; c < C; c++) {
            if (Q8) {
                xq0[c] = *reinterpret_cast<const int4 *>(a.qx + oc(c));
                xsr[c] = a.xs[oc(c) >> 5];
            } else {
                xq0[c] = *reinterpret_cast<const int4 *>(a.qx + oc(c) * 32);
                xq1[c] = *reinterpret_cast<const int4 *>(a.qx + oc(c) * 32 + 16);
                xsr[c] = a.xs[oc(c)];
                xsm[c] = a.xsum[oc(c)];
            }
        }
    } else {
        // straight into LDS (no registers held across the weight loads):
        // each wave fills stripes of 64 pieces, the last stripe's surplus
        // lanes repeat the last piece into the padding after the vector
        const int nq = cols >> 4;
        const int base = wave * 64;
#pragma unroll
        for (int k = 0; k < MQ; k++) {
            const int p0 = base + k * nt;
            if (p0 < nq)  // uniform
                __builtin_amdgcn_global_load_lds(a.qx + 16 * min(p0 + lane, nq - 1), lds_ptr(sqx + 16 * p0), 16, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < MB; k++) {
            const int p0 = base + k * nt;
            if (p0 < nb) {
                __builtin_amdgcn_global_load_lds(a.xs + min(p0 + lane, nb - 1), lds_ptr(sxs + p0), 4, 0, 0);
                if (!Q8) __builtin_amdgcn_global_load_lds(a.xsum + min(p0 + lane, nb - 1), lds_ptr(sxsum + p0), 4, 0, 0);
            }
        }
    }

    // ---- (2) per-row operands of batch j (lane group g = lane / 8 holds
    // row g's), loaded while the batch streams ----
    const int g = lane >> 3, L = lane & 7;
    const int gk = g < K ? g : K - 1;
    float ep0 = 0.0f, cosv = 0.0f, sinv = 0.0f;
    auto load_ops = [&](int j) {
        const int l = min(R0 + j * RB + wave * K + gk, a.rows - 1);
        if (EPI == kEpAdd || EPI == kEpAddCanon) ep0 = *stream_out(a, l);
        if ((EPI == kEpStore || EPI == kEpQKV) && a.bias) ep0 = a.bias[a.row_base + l];
        if (EPI == kEpQKV) {
            const int i0 = a.row_base + (l & ~1);
            const int half = a.hs >> 1;
            int pi = 0;
            if (i0 < a.qdim + a.kvdim) pi = ((i0 < a.qdim ? i0 : i0 - a.qdim) % a.hs) >> 1;
            cosv = a.cos_t[(int64_t)pos * half + pi];
            sinv = a.sin_t[(int64_t)pos * half + pi];
        }
    };

    // ---- (3) the first U chunks of batch 0 ----
    // A row's codes and scales are each a buffer over the row: one lane
    // offset serves every chunk but the last (the chunk's offset is scalar);
    // the last chunk's lane offsets are clamped into the row (lanes past its
    // end re-read its last piece; their blocks are never summed). Past the
    // last batch the same loads go to empty buffers (no records): they
    // return zeros without touching memory, so every batch issues the same
    // loads and the waits stay fixed counts. They still pass through the
    // vector memory queue, which backs up at a launch's start (measured: a
    // 4096x4096 product 5.70 -> 5.17 us without them), so a workgroup of
    // one batch is built without the prefetch (PF false).
    constexpr int NR = (U + C - 1) / C;  // rows the prefetch of a batch's first U chunks reaches
    Row rsrc[K];
    auto set_row = [&](Row &r, int l, bool live) {
        const Src sr = stream_src<EPI>(a, min(l, a.rows - 1), rowbytes, nb);
        r.w = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(sr.w), 0, live ? rowbytes : 0, kRsrcWord3);
        r.s = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(sr.ws), 0, live ? nb * 4 : 0, kRsrcWord3);
    };
#pragma unroll
    for (int h = 0; h < K; h++) set_row(rsrc[h], R0 + wave * K + h, true);
    int4 wb[U];
    float sb[U];
    const int wo = lane * 16;                        // this lane's bytes of a chunk
    const int so = Q8 ? (lane >> 1) * 4 : lane * 4;  // and its block's scale
    constexpr int SPC = Q8 ? 128 : 256;              // scale bytes per chunk
    const int wl = min((C - 1) * 1024 + wo, rowbytes - 16), sl = min((C - 1) * SPC + so, nb * 4 - 4);
    auto load_step = [&](const Row *r, int s, int slot) {
        const int h = s / C, c = s % C;
        const bool last = c == C - 1;
        const rk_v4i v = __builtin_amdgcn_raw_buffer_load_b128(r[h].w, last ? wl : wo, last ? 0 : c * 1024, kAuxStream);
        wb[slot] = make_int4(v.x, v.y, v.z, v.w);
        sb[slot] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r[h].s, last ? sl : so, last ? 0 : c * SPC, 0));
    };
#pragma unroll
    for (int s = 0; s < U; s++) {
        load_step(rsrc, s, s);
        __builtin_amdgcn_sched_barrier(0);  // keep each chunk's codes and scale adjacent in issue order
    }

    // ---- (4) prologue: the input's Q8_0 form into LDS ----
    if (PRO == kProNorm) {
        norm_quant_rt<MG>(xv, wv, cols, nt, a.recip_n, a.norm_eps, sqx, sxs, sxsum,
                          reinterpret_cast<float *>(lds + a.lds_norm), &s_rn);
    } else if (PRO == kProQuant && !XR) {
        // one block a lane from the staged x, once this wave's loads of it
        // are in (issued before its 2U weight loads; the wait is outside the
        // branch so that no path meets the barrier with them pending). The
        // block's eight 16-byte pieces are read from piece l mod 8 on, so a
        // read's lanes fall in distinct banks; the maximum and the code sum
        // do not depend on that order, and each piece's codes go to its place.
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(2 * U));
        const int b = wave * 64 + lane;
        if (b < nb) {
            const float4 *xb4 = reinterpret_cast<const float4 *>(lds + a.lds_norm) + b * 8;
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = xb4[(j + lane) & 7];
            uint32_t pk[8];
            float d;
            int cs;
            quantize_block32(v, pk, d, cs);
            uint32_t *q = reinterpret_cast<uint32_t *>(sqx) + b * 8;
#pragma unroll
            for (int j = 0; j < 8; j++) q[(j + lane) & 7] = pk[j];
            sxs[b] = d;
            sxsum[b] = cs;
        }
    } else if (PRO == kProQuant) {
        // one block per thread (Recip32 once a block)
        if ((int)threadIdx.x < nb) {
            uint32_t pk[8];
            float d;
            int cs;
            quantize_block32(xb, pk, d, cs);
            uint4 *q = reinterpret_cast<uint4 *>(sqx + 32 * threadIdx.x);
            q[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            q[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
            sxs[threadIdx.x] = d;
            sxsum[threadIdx.x] = cs;
        }
    } else if (!XR) {
        // the LDS stores of the loads above: done once no more than the 2U
        // weight loads issued after them are outstanding
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(2 * U));
    }
    if (PRO == kProGlobal && !XR) {
        // The workgroup barrier without __syncthreads' fence: at the fence
        // the compiler counts the direct-to-LDS loads above as pending (it
        // does not see the wait) and would wait for every weight load in
        // flight. This wave's LDS writes are done (the wait above); the
        // memory clobber keeps the LDS reads below after the barrier.
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        asm volatile("s_barrier" ::: "memory");
    } else if (PRO != kProGlobal) {
        __syncthreads();
    }
    if (PRO != kProGlobal && XR) {
#pragma unroll
        for (int c = 0; c < C; c++) {
            if (Q8) {
                xq0[c] = *reinterpret_cast<const int4 *>(sqx + oc(c));
                xsr[c] = sxs[oc(c) >> 5];
            } else {
                xq0[c] = *reinterpret_cast<const int4 *>(sqx + oc(c) * 32);
                xq1[c] = *reinterpret_cast<const int4 *>(sqx + oc(c) * 32 + 16);
                xsr[c] = sxs[oc(c)];
                xsm[c] = sxsum[oc(c)];
            }
        }
    }

    // ---- (5) the batches ----
    const bool has_bias = a.bias != nullptr;
    float best_v = 0.0f;
    int best_i = -1;
    bool nan0 = false;
    for (int j = 0; j < nbatch; j++) {
        // (issued here, after the batch's first U chunks, on every entry to
        // the loop alike, so the waits below are the same fixed counts)
        load_ops(j);
        const bool next = j + 1 < nbatch;  // uniform: the last U chunks prefetch the next batch's first
        Row rn[NR];
        if (PF) {
#pragma unroll
            for (int h = 0; h < NR; h++) set_row(rn[h], R0 + (j + 1) * RB + wave * K + h, next);
        }
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const int h = s / C, c = s % C, slot = s % U;
            float t;
            int b;
            if (Q8) {
                int4 x;
                float xs;
                if (XR) {
                    x = xq0[c];
                    xs = xsr[c];
                } else {
                    x = *reinterpret_cast<const int4 *>(sqx + oc(c));
                    xs = sxs[oc(c) >> 5];
                }
                const int sm = pair_sum(dot16(wb[slot], x, 0));
                t = (float)sm * (sb[slot] * xs);
                b = c * 32 + (lane >> 1);  // only the last chunk can pass the row's last block
                if ((lane & 1) == 0 && (c < C - 1 || b < nb)) tbw[h * rs + (b & 7) * k8p + (b >> 3)] = t;
            } else {
                int4 x0, x1;
                float xs;
                int xsum;
                if (XR) {
                    x0 = xq0[c];
                    x1 = xq1[c];
                    xs = xsr[c];
                    xsum = xsm[c];
                } else {
                    x0 = *reinterpret_cast<const int4 *>(sqx + oc(c) * 32);
                    x1 = *reinterpret_cast<const int4 *>(sqx + oc(c) * 32 + 16);
                    xs = sxs[oc(c)];
                    xsum = sxsum[oc(c)];
                }
                const int4 w = wb[slot];
                const int4 lo = make_int4(w.x & 0x0F0F0F0F, w.y & 0x0F0F0F0F, w.z & 0x0F0F0F0F, w.w & 0x0F0F0F0F);
                const int4 hi =
                    make_int4((int)(((uint32_t)w.x >> 4) & 0x0F0F0F0Fu), (int)(((uint32_t)w.y >> 4) & 0x0F0F0F0Fu),
                              (int)(((uint32_t)w.z >> 4) & 0x0F0F0F0Fu), (int)(((uint32_t)w.w >> 4) & 0x0F0F0F0Fu));
                // nibble j is w_j + 8: sum_b = Σ lo·x_j + Σ hi·x_j+16 - 8·Σ x
                const int sm = dot16(hi, x1, dot16(lo, x0, 0)) - 8 * xsum;
                t = (float)sm * (sb[slot] * xs);
                b = c * 64 + lane;
                if (c < C - 1 || b < nb) tbw[h * rs + (b & 7) * k8p + (b >> 3)] = t;
            }
            if (s + U < NS)
                load_step(rsrc, s + U, slot);
            else if (PF)
                load_step(rn, s + U - NS, slot);
        }
        // the rows: lane group g adds running sum L of row g in block order
        float sum = 0.0f;
        {
            const float *p = tbw + gk * rs + L * k8p;
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
        sum = sum + dppf_x1(sum);
        sum = sum + dppf_x2(sum);
        sum = sum + __int_as_float(dpp_mirror8(__float_as_int(sum)));
        // epilogue: lane 8g writes row g's result
        const int l = R0 + j * RB + wave * K + g;
        const bool valid = g < K && l < a.rows && L == 0;
        if (EPI == kEpQKV || EPI == kEpSilu) {
            const float v = (EPI == kEpQKV && has_bias) ? sum + ep0 : sum;
            const float v1 = __shfl_down(v, 8);  // the pair's second row
            if (valid && (g & 1) == 0) {
                if (EPI == kEpSilu) {
                    const float hv = silu_mul(v, v1);
                    a.seg[0].out[l >> 1] = hv;
                    if (a.qx_out) sh[(l - R0) >> 1] = hv;
                } else {
                    const int i0 = a.row_base + l;
                    float o0 = v, o1 = v1;
                    if (i0 < a.qdim + a.kvdim) {
                        o0 = (v * cosv) - (v1 * sinv);
                        o1 = (v * sinv) + (v1 * cosv);
                    }
                    float *d0 = i0 < a.qdim               ? a.seg[0].out + i0
                                : i0 < a.qdim + a.kvdim ? a.kcache + (int64_t)pos * a.kvdim + (i0 - a.qdim)
                                                        : a.vcache + (int64_t)pos * a.kvdim + (i0 - a.qdim - a.kvdim);
                    d0[0] = o0;
                    d0[1] = o1;  // i0 even: both rows of a pair sit in one of q, k, v
                }
            }
        } else if (valid) {
            float *o = stream_out(a, l);
            if (EPI == kEpStore)
                *o = has_bias ? sum + ep0 : sum;
            else if (EPI == kEpAdd)
                *o = ep0 + sum;
            else if (EPI == kEpAddCanon)
                *o = canonical(ep0 + sum);
            else if (EPI == kEpLogits) {
                *o = sum;
                if (sum == sum)
                    argmax_merge(best_v, best_i, sum, l);
                else if (l == 0)
                    nan0 = true;
            }
        }
        if (PF) {
#pragma unroll
            for (int h = 0; h < K; h++) {
                if (h < NR)
                    rsrc[h] = rn[h];
                else
                    set_row(rsrc[h], R0 + (j + 1) * RB + wave * K + h, next);
            }
        }
    }

    // ---- (6) workgroup epilogues ----
    if (EPI == kEpSilu && a.qx_out) {
        // h's Q8_0 blocks: the launcher gives each workgroup whole blocks
        // (64 logical rows, 32 values of h), eight lanes a block
        __syncthreads();
        const int n = min(a.rows, R0 + a.rows_per_wg) - R0;
        const int np = n >> 1, P0 = R0 >> 1;
        for (int g0 = 0; g0 < (np >> 2); g0 += nt) {  // uniform
            const int gi = g0 + threadIdx.x;
            const int gc = min(gi, (np >> 2) - 1);
            const float4 v = reinterpret_cast<const float4 *>(sh)[gc];
            float d;
            int cs;
            const uint32_t pk = quantize_group(v.x, v.y, v.z, v.w, d, cs);
            if (gi < (np >> 2)) {
                reinterpret_cast<uint32_t *>(a.qx_out + P0)[gi] = pk;
                if ((gi & 7) == 0) {
                    a.xs_out[(P0 >> 5) + (gi >> 3)] = d;
                    a.xsum_out[(P0 >> 5) + (gi >> 3)] = cs;
                }
            }
        }
    }
    if (EPI == kEpLogits) {
        // greedy argmax (internal/llm/sample.go:45-53): over the wave, the
        // workgroup, then one atomicMax of its key into a slot
#pragma unroll
        for (int off = 32; off >= 8; off >>= 1) {
            const float ov = __shfl_down(best_v, off);
            const int oi = __shfl_down(best_i, off);
            argmax_merge(best_v, best_i, ov, oi);
        }
        const bool wnan = __any(nan0);
        if (lane == 0) {
            s_wv[wave] = best_v;
            s_wi[wave] = wnan ? -2 : best_i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float bv = 0.0f;
            int bi = -1;
            bool n0 = false;
            for (int w = 0; w < W; w++) {
                if (s_wi[w] == -2)
                    n0 = true;
                else
                    argmax_merge(bv, bi, s_wv[w], s_wi[w]);
            }
            unsigned long long key = bi < 0 ? 0ull : argmax_key(bv, bi);
            // a NaN first logit makes the argmax 0 (nothing compares above
            // it): the largest key, row 0
            if (n0) key = ~0ull;
            if (key) atomicMax(&a.amax[blockIdx.x % kArgmaxSlots], key);
        }
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Instances and launch.

namespace {

typedef void (*StreamFn)(FusedArgs, int);

struct StreamInst {
    int fmt, pro, epi, k, u, c;
    StreamFn fn, fn1;  // prefetching the next batch; one batch a workgroup
};

#define RK_SI(F, P, E, K, U, C) {F, P, E, K, U, C, stream_kernel<F, P, E, K, U, C, true>, stream_kernel<F, P, E, K, U, C, false>}

// The widths of the configurations this build is measured on (Q8: 2048, 4096 and
// 14336 columns, C = 2, 4 and 14; Q4: 3584/4096 and 18944 columns, C = 2 and
// 10); other widths take fused_kernel.
const StreamInst kStreamInst[] = {
    RK_SI(kFmtQ8, kProQuant, kEpStore, 1, 4, 4),
    RK_SI(kFmtQ8, kProQuant, kEpStore, 2, 4, 4),
    RK_SI(kFmtQ8, kProQuant, kEpStore, 2, 8, 4),
    RK_SI(kFmtQ8, kProNorm, kEpQKV, 2, 8, 4),
    RK_SI(kFmtQ8, kProNorm, kEpSilu, 4, 8, 4),
    RK_SI(kFmtQ8, kProNorm, kEpLogits, 2, 8, 4),
    RK_SI(kFmtQ4, kProNorm, kEpSilu, 4, 8, 2),
    RK_SI(kFmtQ8, kProGlobal, kEpStore, 2, 4, 4),
    RK_SI(kFmtQ8, kProQuant, kEpStore, 1, 7, 14),
    RK_SI(kFmtQ8, kProGlobal, kEpStore, 1, 7, 14),
    RK_SI(kFmtQ8, kProNorm, kEpQKV, 2, 4, 4),
    RK_SI(kFmtQ8, kProGlobal, kEpQKV, 2, 4, 4),
    RK_SI(kFmtQ8, kProGlobal, kEpAdd, 2, 4, 4),
    RK_SI(kFmtQ8, kProNorm, kEpSilu, 4, 4, 4),
    RK_SI(kFmtQ8, kProGlobal, kEpAddCanon, 1, 7, 14),
    RK_SI(kFmtQ8, kProNorm, kEpLogits, 2, 4, 4),
    RK_SI(kFmtQ4, kProNorm, kEpQKV, 2, 4, 2),
    RK_SI(kFmtQ4, kProGlobal, kEpQKV, 2, 4, 2),
    RK_SI(kFmtQ4, kProGlobal, kEpAdd, 2, 4, 2),
    RK_SI(kFmtQ4, kProNorm, kEpSilu, 4, 4, 2),
    RK_SI(kFmtQ4, kProGlobal, kEpAddCanon, 1, 5, 10),
    RK_SI(kFmtQ4, kProQuant, kEpStore, 2, 4, 2),
    RK_SI(kFmtQ4, kProGlobal, kEpStore, 2, 4, 2),
    // 2048 columns (config 5: QKV with the attention RMSNorm, the router,
    // the classifier with the head's RMSNorm)
    RK_SI(kFmtQ8, kProNorm, kEpStore, 2, 4, 2),
    RK_SI(kFmtQ8, kProGlobal, kEpStore, 2, 4, 2),
    RK_SI(kFmtQ8, kProNorm, kEpLogits, 2, 4, 2),
};
#undef RK_SI

// Launch shapes measured on MI355X (256 CUs) for the products of the model
// shapes this build runs: instance (K, U), waves W, batches per workgroup.
struct StreamTune {
    int fmt, pro, epi, rows, cols, k, u, w, nbatch;
};
const StreamTune kStreamTune[] = {
    {kFmtQ8, kProQuant, kEpStore, 4096, 4096, 2, 8, 8, 1},         // config 2
    {kFmtQ8, kProQuant, kEpStore, 14336, 4096, 1, 4, 8, 7},        // config 2
    {kFmtQ8, kProQuant, kEpStore, 4096, 14336, 1, 7, 16, 1},       // config 2
    {kFmtQ8, kProGlobal, kEpStore, 4096, 4096, 2, 4, 4, 1},
    {kFmtQ8, kProGlobal, kEpStore, 14336, 4096, 2, 4, 7, 4},
    {kFmtQ8, kProGlobal, kEpStore, 4096, 14336, 1, 7, 8, 1},
    {kFmtQ8, kProNorm, kEpQKV, 6144, 4096, 2, 4, 12, 1},           // 8B-shape layer
    {kFmtQ8, kProGlobal, kEpAdd, 4096, 4096, 2, 4, 4, 1},
    {kFmtQ8, kProNorm, kEpSilu, 28672, 4096, 4, 8, 8, 2},
    {kFmtQ8, kProGlobal, kEpAddCanon, 4096, 14336, 1, 7, 8, 1},
    {kFmtQ8, kProNorm, kEpLogits, 128256, 4096, 2, 4, 8, 38},
    {kFmtQ4, kProNorm, kEpQKV, 4608, 3584, 2, 4, 9, 1},            // Qwen-7B-shape layer
    {kFmtQ4, kProGlobal, kEpAdd, 3584, 3584, 2, 4, 7, 1},
    {kFmtQ4, kProNorm, kEpSilu, 37888, 3584, 4, 4, 16, 3},
    {kFmtQ4, kProGlobal, kEpAddCanon, 3584, 18944, 1, 5, 8, 1},
    {kFmtQ8, kProNorm, kEpLogits, 152064, 3584, 2, 4, 8, 41},
};

constexpr int kStreamLdsMax = 160 * 1024;

inline int al16(int v) { return (v + 15) & ~15; }

}  // namespace

bool stream_has(int fmt, int pro, int epi, int cols) {
    if (cols <= 0 || cols % 32) return false;
    const int C = fmt == kFmtQ8 ? (cols + 1023) / 1024 : (cols / 32 + 63) / 64;
    for (const StreamInst &i : kStreamInst)
        if (i.fmt == fmt && i.pro == pro && i.epi == epi && i.c == C) return true;
    return false;
}

bool launch_stream(int fmt, int pro, int epi, FusedArgs a, int cu, hipStream_t s) {
    if (a.rows <= 0 || a.cols <= 0 || a.cols % 32) return false;
    const int cols = a.cols, nb = cols / 32;
    const int C = fmt == kFmtQ8 ? (cols + 1023) / 1024 : (nb + 63) / 64;
    if ((epi == kEpAdd || epi == kEpAddCanon || epi == kEpLogits) && a.nseg != 1) return false;
    if (epi == kEpQKV && (a.hs <= 0 || (a.hs & 1) || (a.rows & 1) || (a.row_base & 1) || (a.qdim & 1) || (a.kvdim & 1)))
        return false;
    const bool hq = epi == kEpSilu && a.qx_out;
    if (hq && a.rows % 64) return false;
    if (pro == kProNorm && cols > kMaxNormProCols) return false;

    // Instance and workgroup shape (W waves of K rows a batch, nbatch
    // batches): a measured entry for the shape, else a default.
    const int ncu = cu > 0 ? cu : 256;
    const int wmin = stream_wmin(fmt, pro, C);
    auto find = [&](int k, int u) -> const StreamInst * {
        for (const StreamInst &in : kStreamInst)
            if (in.fmt == fmt && in.pro == pro && in.epi == epi && in.c == C && in.k == k && (u == 0 || in.u == u))
                return &in;
        return nullptr;
    };
    const StreamInst *inst = nullptr;
    int W = 0, nbatch = 0;
    // (an entry below the instance's smallest workgroup is never taken: its
    // prologue would leave part of the input unloaded)
    for (const StreamTune &t : kStreamTune)
        if (t.fmt == fmt && t.pro == pro && t.epi == epi && t.rows == a.rows && t.cols == cols && ncu == 256 &&
            t.w >= wmin && t.w <= 16 && (inst = find(t.k, t.u))) {
            W = t.w;
            nbatch = t.nbatch;
            break;
        }
    if (!inst) {
        // Default: with a prologue per workgroup (quantize, RMSNorm), about
        // one workgroup per CU, as few waves as cover the rows; without,
        // about two per CU of at least four waves.
        for (const StreamInst &in : kStreamInst)
            if (in.fmt == fmt && in.pro == pro && in.epi == epi && in.c == C && (!inst || in.u < inst->u)) inst = &in;
        if (!inst) return false;
        const int K = inst->k;
        const int64_t per_cu = pro == kProGlobal ? 2 : 1;
        const int64_t want = (a.rows + ncu * per_cu - 1) / (ncu * per_cu);  // rows per workgroup
        W = (int)std::min<int64_t>(16, std::max<int64_t>(wmin, (want + K - 1) / K));
        int64_t RB = (int64_t)W * K;
        int64_t nbt = std::max<int64_t>(1, (want + RB - 1) / RB);
        if (hq) {
            while ((64 % RB) && (RB % 64)) RB = (int64_t)(--W) * K;  // a batch divides 64 rows, or 64 divides it
            if (W < wmin) return false;
            nbt = std::max<int64_t>(1, (want + RB - 1) / RB);
            while ((RB * nbt) % 64) nbt++;
        }
        nbatch = (int)nbt;
    }
    const int K = inst->k;
    const int64_t RB = (int64_t)W * K;
    a.rows_per_wg = (int32_t)(RB * nbatch);
    const unsigned grid = (unsigned)((a.rows + a.rows_per_wg - 1) / a.rows_per_wg);

    // LDS: the input's Q8_0 form (codes, scales, code sums), then the terms
    // (the norm's transposed x shares their room), then h.
    const bool xr = fmt == kFmtQ8 ? C <= 4 : C <= 2;
    const int k8p = stream_k8p(fmt, C);
    int at = 0;
    if (pro != kProGlobal || !xr) {
        // whole stripes of 64 pieces (16 bytes of codes, one scale or sum)
        a.lds_xs = (cols + 1023) / 1024 * 1024;
        a.lds_xsum = a.lds_xs + (nb + 63) / 64 * 256;
        at = a.lds_xsum + (nb + 63) / 64 * 256;
    }
    a.lds_res = a.lds_norm = at;
    const int tb = W * K * 8 * k8p * 4;
    // (a wide quantize prologue stages x there: 8 KiB for each wave's 64 blocks)
    at += std::max(tb, pro == kProNorm ? (int)stream_norm_lds(cols) : pro == kProQuant && !xr ? (nb + 63) / 64 * 8192 : 0);
    a.lds_ep = at;
    if (hq) at += al16(a.rows_per_wg / 2 * 4);
    a.lds_bytes = at;
    if (at > kStreamLdsMax) return false;
    const StreamFn fn = nbatch > 1 ? inst->fn : inst->fn1;
    if (at > 64 * 1024) {
        static std::mutex mu;
        std::lock_guard<std::mutex> l(mu);
        (void)hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, kStreamLdsMax);
    }
    RK_LAUNCH(fn, dim3(grid), dim3(64 * W), (size_t)at, s, a, nbatch);
    return true;
}

}  // namespace rk
