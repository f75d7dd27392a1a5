// rk_matvec.hip — Q8_0 / Q4_0 matrix-vector products for gfx950.
//
// Semantics (internal/num/quant.go:14-19, 158-196): the input is quantized
// to Q8_0; block b of a row contributes float32(sum_b)·float32(ws_b·xs_b)
// to running sum b mod 8, in order of b (sums start at +0), and the eight
// sums combine as ((0+1)+(2+3))+((4+5)+(6+7)). sum_b is an exact integer, so
// it is computed with v_dot4 in any order; only the float part is ordered.
//
// Work layout: one wavefront owns a contiguous run of rows and walks each
// row in 1 KiB chunks of weights, one 16-byte (global_load_dwordx4) piece
// per lane, coalesced. Q8: a lane pair holds one 32-byte block; Q4: a lane
// holds one 16-byte block. The block terms of a chunk are gathered into the
// lanes that own the eight running sums (cross-lane moves), which add them
// in block order.
#include "rk_fmath.h"
#include "rk_kernels.h"

namespace rk {

// ---------------------------------------------------------------------------
// Activation quantize: internal/num/quant.go:34-53, eight lanes per block.
__global__ __launch_bounds__(256) void quantize_acts_kernel(const float *__restrict__ x, int64_t nb,
                                                            int8_t *__restrict__ qx, float *__restrict__ xs,
                                                            int32_t *__restrict__ xsum) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t b = t >> 3;
    const bool ok = b < nb;
    float v0 = 0.0f, v1 = 0.0f, v2 = 0.0f, v3 = 0.0f;
    if (ok) {
        const float *p = x + t * 4;
        v0 = p[0];
        v1 = p[1];
        v2 = p[2];
        v3 = p[3];
    }
    // amax = max(|v|) with Go's max; exact in any order.
    float a = gomax(gomax(gomax(0.0f, fabsf(v0)), fabsf(v1)), gomax(fabsf(v2), fabsf(v3)));
    a = gomax(a, __shfl_xor(a, 1));
    a = gomax(a, __shfl_xor(a, 2));
    a = gomax(a, __shfl_xor(a, 4));
    const float d = a * u2f(k1_127);
    const bool zero = (d == 0.0f) || (d != d);
    const float id = recip32(d);
    int c0 = 0, c1 = 0, c2 = 0, c3 = 0;
    if (!zero) {
        c0 = q8_code(v0, id);
        c1 = q8_code(v1, id);
        c2 = q8_code(v2, id);
        c3 = q8_code(v3, id);
    }
    int s = c0 + c1 + c2 + c3;
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if (ok) {
        const uint32_t packed = (uint32_t)(c0 & 255) | ((uint32_t)(c1 & 255) << 8) | ((uint32_t)(c2 & 255) << 16) |
                                ((uint32_t)(c3 & 255) << 24);
        reinterpret_cast<uint32_t *>(qx)[t] = packed;
        if ((threadIdx.x & 7) == 0) {
            xs[b] = d;
            xsum[b] = s;
        }
    }
}

void launch_quantize_acts(const float *x, int64_t n, int8_t *qx, float *xs, int32_t *xsum, hipStream_t s) {
    const int64_t nb = n / 32;
    if (nb <= 0) return;
    const int64_t threads = nb * 8;
    RK_LAUNCH(quantize_acts_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, x, nb, qx, xs,
                       xsum);
}

// ---------------------------------------------------------------------------
// Matrix-vector products.
//
// Each wavefront owns a contiguous run of rows and walks them in chunks of
// 1 KiB of codes (one 16-byte piece per lane). The loads of the next chunk
// (codes, their scales, and the matching quantized input and its scales) are
// issued before the current chunk is consumed, so every wave keeps a chunk in
// flight; the quantized input comes through the same loads (it stays in L1/
// L2), not LDS, so the wait for the current chunk never waits on later ones.
// Waves per CU are as many as registers allow: that, not deeper per-wave
// prefetch, is what fills HBM (measured on MI355X).

constexpr int kWaves = 4;  // wavefronts per workgroup

struct RowRef {
    const uint8_t *w;
    const float *ws;
    float *out;
    int64_t r;
};

// The matrix (segment) holding global row g, and the row within it. The
// segment table is indexed with uniform compares, not a dynamic index, so it
// stays in kernel-argument registers.
__device__ __forceinline__ RowRef locate(const MatvecArgs &a, int64_t g) {
    RowRef x{a.seg[0].w, a.seg[0].ws, a.seg[0].out, g};
    if (a.nseg > 1 && x.r >= a.seg[0].rows) {
        x.r -= a.seg[0].rows;
        x.w = a.seg[1].w; x.ws = a.seg[1].ws; x.out = a.seg[1].out;
        if (a.nseg > 2 && x.r >= a.seg[1].rows) {
            x.r -= a.seg[1].rows;
            x.w = a.seg[2].w; x.ws = a.seg[2].ws; x.out = a.seg[2].out;
            if (a.nseg > 3 && x.r >= a.seg[2].rows) {
                x.r -= a.seg[2].rows;
                x.w = a.seg[3].w; x.ws = a.seg[3].ws; x.out = a.seg[3].out;
            }
        }
    }
    return x;
}

// Exact integer sum of a lane pair (quad_perm [1,0,3,2]).
__device__ __forceinline__ int pair_sum(int s) { return s + __builtin_amdgcn_mov_dpp(s, 0xB1, 0xF, 0xF, false); }

__device__ __forceinline__ int dot16(int4 w, int4 x, int acc) {
    acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
    acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
    acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
    acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
    return acc;
}

// Rows of this wave: a contiguous run, [r0, r1).
__device__ __forceinline__ bool wave_rows(int64_t total, int64_t per, int64_t &r0, int64_t &r1) {
    const int64_t wave = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    r0 = wave * per;
    r1 = r0 + per < total ? r0 + per : total;
    return r0 < r1;
}

// The row's result: stored, or added to what the output holds (a residual
// connection, x += W·v, internal/llm/model.go:596-598, 608-610), made
// canonical if asked.
__device__ __forceinline__ void put_row(const MatvecArgs &a, float *out, float res) {
    if (a.epilogue == kEpiStore) {
        *out = res;
    } else {
        const float v = *out + res;
        *out = a.epilogue == kEpiAddCanonical ? canonical(v) : v;
    }
}

// One chunk's operands for one lane.
struct Q8Chunk {
    int4 w, x;
    float ws, xs;
};

// Q8_0: chunk c of a row is blocks [32c, 32c+32); lane pair k = lane/2 holds
// block 32c+k. Running sum L (0..7) lives in lane 2L; in chunk c it takes the
// blocks 32c+L, +8, +16, +24, held by lanes 2L, 2L+16, 2L+32, 2L+48.
__global__ __launch_bounds__(256) void matvec_q8_kernel(MatvecArgs a) {
    int64_t r0, r1;
    if (!wave_rows(a.total_rows, a.per_wave, r0, r1)) return;
    const int lane = threadIdx.x & 63;
    const int cols = a.cols, nb = cols >> 5;
    const int C = (cols + 1023) >> 10;
    const int64_t nsteps = (r1 - r0) * C;

    int64_t lg = r0, pg = r0;  // load / process cursors: global row, chunk
    int lc = 0, pc = 0;
    auto load = [&](Q8Chunk &k) {
        k.w = k.x = make_int4(0, 0, 0, 0);
        k.ws = k.xs = 0.0f;
        const RowRef rr = locate(a, lg);
        const int off = lc * 1024 + lane * 16;
        if (off < cols) {
            k.w = *reinterpret_cast<const int4 *>(rr.w + rr.r * cols + off);
            k.ws = rr.ws[rr.r * nb + (off >> 5)];
            k.x = *reinterpret_cast<const int4 *>(a.qx + off);
            k.xs = a.xs[off >> 5];
        }
        if (++lc == C) {
            lc = 0;
            ++lg;
        }
    };
    float acc = 0.0f;
    auto process = [&](const Q8Chunk &k) {
        const int s = pair_sum(dot16(k.w, k.x, 0));
        const float t = (float)s * (k.ws * k.xs);
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
        if (++pc == C) {
            // sums in lanes 0,2,..,14: ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7))
            const float p2 = acc + __shfl_down(acc, 2);
            const float q4 = p2 + __shfl_down(p2, 4);
            const float res = q4 + __shfl_down(q4, 8);
            if (lane == 0) {
                const RowRef rr = locate(a, pg);
                put_row(a, rr.out + rr.r, res);
            }
            acc = 0.0f;
            pc = 0;
            ++pg;
        }
    };
    Q8Chunk ka, kb;
    load(ka);
    for (int64_t st = 0; st < nsteps;) {
        if (st + 1 < nsteps) load(kb);
        process(ka);
        if (++st >= nsteps) break;
        if (st + 1 < nsteps) load(ka);
        process(kb);
        ++st;
    }
}

struct Q4Chunk {
    int4 w, x0, x1;
    float ws, xs;
    int xsum;
};

// Q4_0: a row has cols/2 bytes; chunk c is blocks [64c, 64c+64), lane l
// holds block 64c+l (16 bytes: byte j = element j low, j+16 high, +8).
// sum_b = sum(lo_j·x_j) + sum(hi_j·x_{j+16}) - 8·sum(x): exact. Running sum
// L lives in lane L and takes lanes L, L+8, ..., L+56 in order.
__global__ __launch_bounds__(256) void matvec_q4_kernel(MatvecArgs a) {
    int64_t r0, r1;
    if (!wave_rows(a.total_rows, a.per_wave, r0, r1)) return;
    const int lane = threadIdx.x & 63;
    const int cols = a.cols, nb = cols >> 5;
    const int rowb = cols >> 1;
    const int C = (nb + 63) >> 6;
    const int64_t nsteps = (r1 - r0) * C;

    int64_t lg = r0, pg = r0;
    int lc = 0, pc = 0;
    auto load = [&](Q4Chunk &k) {
        k.w = k.x0 = k.x1 = make_int4(0, 0, 0, 0);
        k.ws = k.xs = 0.0f;
        k.xsum = 0;
        const RowRef rr = locate(a, lg);
        const int blk = lc * 64 + lane;
        if (blk < nb) {
            k.w = *reinterpret_cast<const int4 *>(rr.w + rr.r * rowb + blk * 16);
            k.ws = rr.ws[rr.r * nb + blk];
            k.x0 = *reinterpret_cast<const int4 *>(a.qx + blk * 32);
            k.x1 = *reinterpret_cast<const int4 *>(a.qx + blk * 32 + 16);
            k.xs = a.xs[blk];
            k.xsum = a.xsum[blk];
        }
        if (++lc == C) {
            lc = 0;
            ++lg;
        }
    };
    float acc = 0.0f;
    auto process = [&](const Q4Chunk &k) {
        const int4 w = k.w;
        const int4 lo = make_int4(w.x & 0x0F0F0F0F, w.y & 0x0F0F0F0F, w.z & 0x0F0F0F0F, w.w & 0x0F0F0F0F);
        const int4 hi = make_int4((int)(((uint32_t)w.x >> 4) & 0x0F0F0F0Fu), (int)(((uint32_t)w.y >> 4) & 0x0F0F0F0Fu),
                                  (int)(((uint32_t)w.z >> 4) & 0x0F0F0F0Fu), (int)(((uint32_t)w.w >> 4) & 0x0F0F0F0Fu));
        const int s = dot16(hi, k.x1, dot16(lo, k.x0, 0)) - 8 * k.xsum;
        const float t = (float)s * (k.ws * k.xs);
        float tj[8];
        tj[0] = t;
#pragma unroll
        for (int j = 1; j < 8; ++j) tj[j] = __shfl_down(t, 8 * j);
        if (lane < 8) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (pc * 64 + lane + 8 * j < nb) acc += tj[j];
        }
        if (++pc == C) {
            const float p2 = acc + __shfl_down(acc, 1);
            const float q4 = p2 + __shfl_down(p2, 2);
            const float res = q4 + __shfl_down(q4, 4);
            if (lane == 0) {
                const RowRef rr = locate(a, pg);
                put_row(a, rr.out + rr.r, res);
            }
            acc = 0.0f;
            pc = 0;
            ++pg;
        }
    };
    Q4Chunk ka, kb;
    load(ka);
    for (int64_t st = 0; st < nsteps;) {
        if (st + 1 < nsteps) load(kb);
        process(ka);
        if (++st >= nsteps) break;
        if (st + 1 < nsteps) load(ka);
        process(kb);
        ++st;
    }
}

// Grid: about 64 waves per CU requested (residency is then set by
// registers), each owning a contiguous run of rows.
static unsigned matvec_grid(MatvecArgs &a, int cu) {
    const int64_t target = (int64_t)(cu > 0 ? cu : 256) * 64;
    a.per_wave = (a.total_rows + target - 1) / target;
    const int64_t waves = (a.total_rows + a.per_wave - 1) / a.per_wave;
    return (unsigned)((waves + kWaves - 1) / kWaves);
}

void launch_matvec_q8(const MatvecArgs &args, int cu, hipStream_t s) {
    if (args.total_rows <= 0) return;
    MatvecArgs a = args;
    const unsigned grid = matvec_grid(a, cu);
    RK_LAUNCH(matvec_q8_kernel, dim3(grid), dim3(64 * kWaves), 0, s, a);
}

void launch_matvec_q4(const MatvecArgs &args, int cu, hipStream_t s) {
    if (args.total_rows <= 0) return;
    MatvecArgs a = args;
    const unsigned grid = matvec_grid(a, cu);
    RK_LAUNCH(matvec_q4_kernel, dim3(grid), dim3(64 * kWaves), 0, s, a);
}

}  // namespace rk
