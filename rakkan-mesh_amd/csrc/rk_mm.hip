// rk_mm.hip — batched quantized products for prompt prefill, on gfx950's
// int8 matrix cores. The reference runs a prompt one token at a time
// (internal/llm/model.go:504-518), each token's products through MatVecQ8/Q4
// (internal/num/quant.go:158-196); a batch here gives every (token, row) the
// bits of that token's own product:
//
//   out[t][r] = ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7)),
//   s_(b mod 8) += float32(sum_b[r][t])·float32(ws[r][b]·xs[t][b]) in order of b,
//
// with sum_b the exact integer dot of block b. One v_mfma_i32_16x16x32_i8
// (K = 32 = one block, accumulator zero) gives sum_b for 16 rows × 16 tokens;
// the f32 steps above then run on the vector ALUs in that order, so those
// four operations per (row, token, block) bound the kernel, not the MFMA.
//
// Work layout: a workgroup (eight waves) owns 64 rows × 64 tokens and
// walks the blocks in chunks of eight (one per running sum). A chunk's codes
// and scales are staged in LDS (Q4_0 unpacked to signed codes once there),
// double-buffered: the next chunk's global loads are in flight while the
// current one is multiplied. Tiles are numbered so that each XCD takes a
// contiguous run, keeping a row tile's token tiles on one L2.
#include <mutex>

#include "rk_dev.h"
#include "rk_mm.h"

namespace rk {

namespace {

constexpr int kMmRows = 64;      // output rows per workgroup (kEpSilu: 32 rows of W1 and of W3)
constexpr int kMmToks = 64;      // tokens per workgroup
constexpr int kMmKB = 8;         // blocks per staged chunk, one per running sum
constexpr int kMmThreads = 512;  // eight waves
// Bytes per staged row: 16 rows read at one offset fall in distinct banks.
constexpr int kMmPitch = kMmKB * 32 + 8;
constexpr int kHbPitch = 36;  // kEpSilu: floats per token row of h

struct MmStage {
    int8_t w[kMmRows][kMmPitch];  // codes of the staged rows (Q4 unpacked)
    int8_t x[kMmToks][kMmPitch];  // codes of the staged tokens
    float ws[kMmKB][kMmRows];     // weight scales, block-major
    float xs[kMmKB][kMmToks];     // input scales, block-major
};
static_assert(sizeof(MmStage) % 16 == 0, "stage buffers stay 16-byte aligned");
static_assert(kMmToks * kHbPitch * 4 <= (int)sizeof(MmStage), "h tile fits a stage buffer");

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

// 16 bytes into LDS that is 8-byte aligned (staged rows have an odd count
// of 8-byte units).
__device__ __forceinline__ void lds_put16(int8_t *p, v4i v) {
    reinterpret_cast<v2i *>(p)[0] = v2i{v.x, v.y};
    reinterpret_cast<v2i *>(p)[1] = v2i{v.z, v.w};
}

// Four Q4 nibbles (0..15, one per byte) to their signed codes n-8 (one per
// byte): the OR keeps every byte >= 8 so the subtraction borrows nowhere.
__device__ __forceinline__ uint32_t nib_signed(uint32_t n) { return ((n | 0x80808080u) - 0x08080808u) ^ 0x80808080u; }

// Source of logical output row g (< rows): segment and row in it. The
// segment is returned by value, its fields picked with selects: a reference
// into the kernel-argument array under a lane-varying index made the
// compiler copy the arguments to scratch and pick a wrong segment for some
// lanes of a three-segment launch.
__device__ __forceinline__ MatSeg seg_of(const MmArgs &a, int g, int &r) {
    r = g;
    const bool in1 = a.nseg > 1 && r >= a.seg[0].rows;
    if (in1) r -= (int)a.seg[0].rows;
    const bool in2 = in1 && a.nseg > 2 && r >= a.seg[1].rows;
    if (in2) r -= (int)a.seg[1].rows;
    MatSeg s;
    s.w = in2 ? a.seg[2].w : in1 ? a.seg[1].w : a.seg[0].w;
    s.ws = in2 ? a.seg[2].ws : in1 ? a.seg[1].ws : a.seg[0].ws;
    s.out = in2 ? a.seg[2].out : in1 ? a.seg[1].out : a.seg[0].out;
    s.rows = in2 ? a.seg[2].rows : in1 ? a.seg[1].rows : a.seg[0].rows;
    return s;
}

}  // namespace

template <int FMT, int EPI>
__global__ __launch_bounds__(kMmThreads) void mm_kernel(MmArgs a) {
    extern __shared__ __align__(16) char lds[];
    MmStage *stg = reinterpret_cast<MmStage *>(lds);  // two buffers
    constexpr bool SILU = EPI == kEpSilu;
    // A wave's tiles of 16 rows x 16 tokens: one row tile and two token
    // tiles, or (kEpSilu) the same rows of W1 and of W3 and one token tile.
    constexpr int TI = SILU ? 2 : 1, TJ = SILU ? 1 : 2;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lq = lane >> 4, ln = lane & 15;
    const int cols = a.cols, nb = cols >> 5, T = a.tokens;
    const int rowbytes = FMT == kFmtQ8 ? cols : cols >> 1;

    // this workgroup's tile: XCD x (workgroups x, x+8, ...) takes tiles
    // [x·per, (x+1)·per), row-tile major
    const int ntr = SILU ? (a.rows + 31) >> 5 : (a.rows + kMmRows - 1) / kMmRows;
    const int ntt = (T + kMmToks - 1) / kMmToks;
    const int total = ntr * ntt;
    const int per = (total + 7) >> 3;
    const int tile = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (tile >= total) return;
    const int rt = tile / ntt, tt = tile - rt * ntt;
    const int row0 = rt * (SILU ? 32 : kMmRows);
    const int tok0 = tt * kMmToks;

    // staged row m -> its codes and scales (rows past the end clamped: their
    // results are never stored)
    auto row_src = [&](int m, const uint8_t *&w, const float *&ws) __attribute__((always_inline)) {
        int r;
        MatSeg s;
        if (SILU) {
            r = min(row0 + (m & 31), a.rows - 1);
            s = m < 32 ? a.seg[0] : a.seg[1];
        } else {
            s = seg_of(a, min(row0 + m, a.rows - 1), r);
        }
        w = s.w + (int64_t)r * rowbytes;
        ws = s.ws + (int64_t)r * nb;
    };

    // ---- staging: each thread's rows and tokens, fixed for the kernel ----
    // Q8 codes: 16-byte piece p = tid + 512j of the chunk's 64 rows x 256
    // bytes (row p>>4, piece p&15); Q4: piece tid of 64 rows x 8 blocks (row
    // tid>>3, block tid&7); inputs like Q8 codes. Scales: row (or token)
    // tid>>3, block tid&7.
    constexpr int NW = FMT == kFmtQ8 ? 2 : 1;
    const uint8_t *wrow[NW];
    const float *wsrow;
    const uint8_t *unused_w;
    const float *unused_ws;
#pragma unroll
    for (int j = 0; j < NW; j++) row_src(FMT == kFmtQ8 ? (tid >> 4) + 32 * j : tid >> 3, wrow[j], unused_ws);
    row_src(tid >> 3, unused_w, wsrow);
    const int8_t *xrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) xrow[j] = a.qx + (int64_t)min(tok0 + (tid >> 4) + 32 * j, T - 1) * cols;
    const float *xsrow = a.xs + (int64_t)min(tok0 + (tid >> 3), T - 1) * nb;

    const int nchunks = (nb + kMmKB - 1) / kMmKB;
    v4i rw[NW], rx[2];
    float rws, rxs;
    // loads of the chunk starting at block c (past the last chunk: the last
    // chunk again; blocks past nb read the last block: never used)
    auto stage_load = [&](int c) __attribute__((always_inline)) {
        c = min(c, (nchunks - 1) * kMmKB);
        const int o = min(c * 32 + (tid & 15) * 16, cols - 16);
        const int bk = min(c + (tid & 7), nb - 1);
#pragma unroll
        for (int j = 0; j < NW; j++) {
            if (FMT == kFmtQ8)
                rw[j] = *reinterpret_cast<const v4i *>(wrow[j] + o);
            else
                rw[j] = *reinterpret_cast<const v4i *>(wrow[j] + bk * 16);
        }
#pragma unroll
        for (int j = 0; j < 2; j++) rx[j] = *reinterpret_cast<const v4i *>(xrow[j] + o);
        rws = wsrow[bk];
        rxs = xsrow[bk];
    };
    auto stage_store = [&](MmStage &S) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NW; j++) {
            if (FMT == kFmtQ8) {
                lds_put16(&S.w[(tid >> 4) + 32 * j][(tid & 15) * 16], rw[j]);
            } else {
                // byte i of the block: low nibble w_i, high nibble w_(i+16)
                const v4i v = rw[j];
                const v4i lo = v4i{(int)nib_signed(v.x & 0x0F0F0F0Fu), (int)nib_signed(v.y & 0x0F0F0F0Fu),
                                   (int)nib_signed(v.z & 0x0F0F0F0Fu), (int)nib_signed(v.w & 0x0F0F0F0Fu)};
                const v4i hi = v4i{(int)nib_signed(((uint32_t)v.x >> 4) & 0x0F0F0F0Fu),
                                   (int)nib_signed(((uint32_t)v.y >> 4) & 0x0F0F0F0Fu),
                                   (int)nib_signed(((uint32_t)v.z >> 4) & 0x0F0F0F0Fu),
                                   (int)nib_signed(((uint32_t)v.w >> 4) & 0x0F0F0F0Fu)};
                int8_t *dst = &S.w[tid >> 3][(tid & 7) * 32];
                lds_put16(dst, lo);
                lds_put16(dst + 16, hi);
            }
        }
#pragma unroll
        for (int j = 0; j < 2; j++) lds_put16(&S.x[(tid >> 4) + 32 * j][(tid & 15) * 16], rx[j]);
        S.ws[tid & 7][tid >> 3] = rws;
        S.xs[tid & 7][tid >> 3] = rxs;
    };

    // ---- products ----
    // A lane holds, per tile, token tb(tj) + ln and rows rb(ti) + 4·lq + i,
    // i < 4 (the MFMA's 16x16 result layout).
    const int wr = SILU ? (wave & 1) : (wave & 3);
    const int wt = SILU ? (wave >> 1) : (wave >> 2);
    auto rb = [&](int ti) { return SILU ? 32 * ti + 16 * wr : 16 * wr; };
    auto tb = [&](int tj) { return SILU ? 16 * wt : 32 * wt + 16 * tj; };
    float acc[TI][TJ][kMmKB][4];
#pragma unroll
    for (int ti = 0; ti < TI; ti++)
#pragma unroll
        for (int tj = 0; tj < TJ; tj++)
#pragma unroll
            for (int k = 0; k < kMmKB; k++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[ti][tj][k][i] = 0.0f;

    // Block k of the staged chunk in three steps: its operand reads from LDS
    // (kload), its MFMAs (kmma), its terms into running sum k (kterms). A
    // chunk runs them two blocks apart: block k+2's reads and block k+1's
    // MFMAs are issued before block k's terms, so neither the LDS nor the
    // matrix results are waited for.
    struct KOps {
        long fa[TI], fb[TJ];
        float4 wsv[TI];
        float xsv[TJ];
    };
    struct KRes {
        v4i d[TI][TJ];
        float4 wsv[TI];
        float xsv[TJ];
    };
    auto kload = [&](const MmStage &S, int k, KOps &o) __attribute__((always_inline)) {
#pragma unroll
        for (int ti = 0; ti < TI; ti++) o.fa[ti] = *reinterpret_cast<const long *>(&S.w[rb(ti) + ln][k * 32 + 8 * lq]);
#pragma unroll
        for (int tj = 0; tj < TJ; tj++) o.fb[tj] = *reinterpret_cast<const long *>(&S.x[tb(tj) + ln][k * 32 + 8 * lq]);
#pragma unroll
        for (int ti = 0; ti < TI; ti++) o.wsv[ti] = *reinterpret_cast<const float4 *>(&S.ws[k][rb(ti) + 4 * lq]);
#pragma unroll
        for (int tj = 0; tj < TJ; tj++) o.xsv[tj] = S.xs[k][tb(tj) + ln];
    };
    auto kmma = [&](const KOps &o, KRes &r) __attribute__((always_inline)) {
#pragma unroll
        for (int ti = 0; ti < TI; ti++)
#pragma unroll
            for (int tj = 0; tj < TJ; tj++)
                r.d[ti][tj] = __builtin_amdgcn_mfma_i32_16x16x32_i8(o.fa[ti], o.fb[tj], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int ti = 0; ti < TI; ti++) r.wsv[ti] = o.wsv[ti];
#pragma unroll
        for (int tj = 0; tj < TJ; tj++) r.xsv[tj] = o.xsv[tj];
    };
    auto kterms = [&](const KRes &r, int k) __attribute__((always_inline)) {
#pragma unroll
        for (int ti = 0; ti < TI; ti++) {
            const float w4[4] = {r.wsv[ti].x, r.wsv[ti].y, r.wsv[ti].z, r.wsv[ti].w};
#pragma unroll
            for (int tj = 0; tj < TJ; tj++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[ti][tj][k][i] += (float)r.d[ti][tj][i] * (w4[i] * r.xsv[tj]);
        }
    };
    // blocks 0..n-1 of a staged chunk, pipelined as above
    auto chunk = [&](const MmStage &S, int n) __attribute__((always_inline)) {
        KOps o[2];
        KRes r[2];
        kload(S, 0, o[0]);
        if (n > 1) kload(S, 1, o[1]);
        kmma(o[0], r[0]);
#pragma unroll
        for (int k = 0; k < kMmKB; k++) {
            if (k + 2 < n) kload(S, k + 2, o[k & 1]);
            if (k + 1 < n) kmma(o[(k + 1) & 1], r[(k + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
            if (k < n) kterms(r[k & 1], k);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Whole chunks in one loop of one path (a second path inside the loop
    // makes the compiler copy all 64 running sums at every iteration), then
    // the short last chunk, if any, after it.
    const int nfull = nb / kMmKB;
    stage_load(0);
    stage_store(stg[0]);
    __syncthreads();
    for (int ci = 0; ci < nfull; ci++) {
        // the next chunk's loads (past the last chunk they re-read it and
        // fill the idle buffer, which nothing reads)
        stage_load((ci + 1) * kMmKB);
        chunk(stg[ci & 1], kMmKB);
        stage_store(stg[(ci + 1) & 1]);
        __syncthreads();
    }
    if (nfull < nchunks) chunk(stg[nfull & 1], nb - nfull * kMmKB);  // absent blocks are skipped, not added as zeros

    // ---- results: the fixed tree of the eight running sums, then the
    // epilogue per (row, token) ----
    float res[TI][TJ][4];
#pragma unroll
    for (int ti = 0; ti < TI; ti++)
#pragma unroll
        for (int tj = 0; tj < TJ; tj++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float p0 = acc[ti][tj][0][i] + acc[ti][tj][1][i], p1 = acc[ti][tj][2][i] + acc[ti][tj][3][i];
                const float p2 = acc[ti][tj][4][i] + acc[ti][tj][5][i], p3 = acc[ti][tj][6][i] + acc[ti][tj][7][i];
                res[ti][tj][i] = (p0 + p1) + (p2 + p3);
            }

    if (SILU) {
        // h = silu(W1·x)·(W3·x) into LDS [token][32 rows] (over stage
        // buffer 0, once every wave is past its last read of it), then each
        // token's 32 values (one Q8_0 block of h) quantized by eight lanes
        float *hb = reinterpret_cast<float *>(lds);
        __syncthreads();
        float4 h4;
        h4.x = silu_mul(res[0][0][0], res[1][0][0]);
        h4.y = silu_mul(res[0][0][1], res[1][0][1]);
        h4.z = silu_mul(res[0][0][2], res[1][0][2]);
        h4.w = silu_mul(res[0][0][3], res[1][0][3]);
        *reinterpret_cast<float4 *>(&hb[(tb(0) + ln) * kHbPitch + 16 * wr + 4 * lq]) = h4;
        __syncthreads();
        const int nbh = a.rows >> 5;
        static_assert(kMmToks * 8 == kMmThreads, "one quantizer task per thread");
        const int n = tid >> 3, g = tid & 7;
        const float4 v = *reinterpret_cast<const float4 *>(&hb[n * kHbPitch + 4 * g]);
        float dsc;
        int cs;
        const uint32_t pk = quantize_group(v.x, v.y, v.z, v.w, dsc, cs);
        const int t = tok0 + n;
        if (t < T) {
            reinterpret_cast<uint32_t *>(a.qx_out + (int64_t)t * a.rows + row0)[g] = pk;
            if (g == 0) {
                a.xs_out[(int64_t)t * nbh + (row0 >> 5)] = dsc;
                a.xsum_out[(int64_t)t * nbh + (row0 >> 5)] = cs;
            }
        }
        return;
    }

#pragma unroll
    for (int tj = 0; tj < TJ; tj++) {
        const int t = tok0 + tb(tj) + ln;
        if (t >= T) continue;
#pragma unroll
        for (int ti = 0; ti < TI; ti++) {
            const int gb = row0 + rb(ti) + 4 * lq;  // the lane's first row
            if (EPI == kEpQKV) {
                const int pos = a.seq_pos ? a.seq_pos[t] : a.pos0 + t, half = a.hs >> 1;
                const int64_t cache0 = (int64_t)t * a.cache_stride;  // token t's sequence's caches
#pragma unroll
                for (int pr = 0; pr < 2; pr++) {
                    const int g0 = gb + 2 * pr;  // an even row: a rotary pair with g0 + 1
                    const int l0 = a.row_base + g0;  // its logical q/k/v row
                    float v0 = res[ti][tj][2 * pr], v1 = res[ti][tj][2 * pr + 1];
                    if (a.bias) {
                        v0 = v0 + a.bias[a.row_base + min(g0, a.rows - 1)];
                        v1 = v1 + a.bias[a.row_base + min(g0 + 1, a.rows - 1)];
                    }
                    if (l0 < a.qdim + a.kvdim) {
                        const int ih = l0 < a.qdim ? l0 : l0 - a.qdim;
                        const int pi = (ih % a.hs) >> 1;
                        const float co = a.cos_t[(int64_t)pos * half + pi], si = a.sin_t[(int64_t)pos * half + pi];
                        const float r0 = (v0 * co) - (v1 * si);
                        const float r1 = (v0 * si) + (v1 * co);
                        v0 = r0;
                        v1 = r1;
                    }
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        if (g0 + h >= a.rows) continue;
                        const int l = l0 + h;
                        float *dst = l < a.qdim ? a.q + (int64_t)t * a.qdim + l
                                     : l < a.qdim + a.kvdim
                                         ? a.kcache + cache0 + (int64_t)pos * a.kvdim + (l - a.qdim)
                                         : a.vcache + cache0 + (int64_t)pos * a.kvdim + (l - a.qdim - a.kvdim);
                        *dst = h ? v1 : v0;
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int g = gb + i;
                    if (g >= a.rows) continue;
                    const float v = res[ti][tj][i];
                    if (EPI == kEpStore) {
                        int r;
                        const MatSeg s = seg_of(a, g, r);
                        s.out[(int64_t)t * s.rows + r] = a.bias ? v + a.bias[g] : v;
                    } else if (EPI == kEpAdd) {
                        float *p = a.x + (int64_t)t * a.ldx + g;
                        *p = *p + v;
                    } else if (EPI == kEpAddCanon) {
                        float *p = a.x + (int64_t)t * a.ldx + g;
                        *p = canonical(*p + v);
                    }
                }
            }
        }
    }
}

// ---- Small batches (up to kRowsMaxT tokens) of Q8 rows ----
// A 64-token tile wastes most of its work on a few tokens and leaves a
// product with few row tiles on few CUs. Here eight lanes hold a row's
// blocks in registers, lane l of the eight the blocks l, l+8, ... (pieces of
// 64 blocks at a time), and keep MatVecQ8's running sum l for each of the
// workgroup's TPG tokens, whose codes and scales are staged in LDS (every
// group of a wave reads the same input bytes at once: an LDS broadcast);
// tree8 then gives each (row, token) the bits of its own product. A
// workgroup owns 32 rows and one run of TPG tokens; the runs of a row tile
// are adjacent on one XCD, so its rows come from HBM once.
constexpr int kRowsThreads = 256;
constexpr int kRowsPerWg = kRowsThreads / 8;
constexpr int kRowsMaxT = 16;

__host__ __device__ constexpr int rows_lds(int tpg, int cols) { return tpg * cols + tpg * (cols / 32) * 4; }

template <int EPI, int TPG>
__global__ __launch_bounds__(kRowsThreads) void mm_rows_kernel(MmArgs a, int ntg) {
    extern __shared__ __align__(16) char lds[];
    const int tid = threadIdx.x, grp = tid >> 3, rl = tid & 7;
    const int cols = a.cols, nb = cols >> 5, T = a.tokens;
    const int nrt = (a.rows + kRowsPerWg - 1) / kRowsPerWg;
    const int total = nrt * ntg;
    const int per = (total + 7) >> 3;
    const int tile = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (tile >= total) return;
    const int rt = tile / ntg, tg = tile - rt * ntg;
    const int tok0 = tg * TPG, nt = min(TPG, T - tok0);

    int8_t *xq = reinterpret_cast<int8_t *>(lds);                 // [nt][cols] codes
    float *xsc = reinterpret_cast<float *>(lds + (size_t)TPG * cols);  // [nt][nb] scales
    {
        const int4 *src = reinterpret_cast<const int4 *>(a.qx + (int64_t)tok0 * cols);
        const int np = nt * (cols >> 4);
        for (int p = tid; p < np; p += kRowsThreads) reinterpret_cast<int4 *>(xq)[p] = src[p];
        const float *ssrc = a.xs + (int64_t)tok0 * nb;
        for (int p = tid; p < nt * nb; p += kRowsThreads) xsc[p] = ssrc[p];
    }
    __syncthreads();

    const int g = rt * kRowsPerWg + grp;  // the group's output row
    int r;
    const MatSeg sg = seg_of(a, min(g, a.rows - 1), r);
    const uint8_t *row = sg.w + (int64_t)r * cols;
    const float *rs = sg.ws + (int64_t)r * nb;
    float acc[TPG];
#pragma unroll
    for (int t = 0; t < TPG; t++) acc[t] = 0.0f;
    for (int p0 = 0; p0 < nb; p0 += 64) {  // pieces of 64 blocks: each lane's eight
        int4 c0[8], c1[8];
        float sw[8];
        lane_row_load<8, false>(c0, c1, sw, row + 32 * p0, rs + p0, nb - p0, rl);
#pragma unroll
        for (int t = 0; t < TPG; t++)
            if (t < nt)
                acc[t] = lane_running_sum_from<8>(acc[t], c0, c1, sw, xq + (size_t)t * cols + 32 * p0,
                                                  xsc + t * nb + p0, nb - p0, rl);
    }
#pragma unroll
    for (int t = 0; t < TPG; t++) acc[t] = tree8(acc[t]);
    if (g >= a.rows) return;
#pragma unroll
    for (int t = 0; t < TPG; t++) {
        if ((t & 7) != rl || t >= nt) continue;  // lane l stores tokens l, l+8
        const float v = acc[t];
        const int tk = tok0 + t;
        if (EPI == kEpStore) {
            sg.out[(int64_t)tk * sg.rows + r] = a.bias ? v + a.bias[g] : v;
        } else if (EPI == kEpAdd) {
            float *p = a.x + (int64_t)tk * a.ldx + g;
            *p = *p + v;
        } else if (EPI == kEpAddCanon) {
            float *p = a.x + (int64_t)tk * a.ldx + g;
            *p = canonical(*p + v);
        }
    }
}

template <int EPI, int TPG>
static void launch_rows_one(const MmArgs &a, int ntg, unsigned grid, hipStream_t s) {
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute((const void *)mm_rows_kernel<EPI, TPG>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    RK_LAUNCH((mm_rows_kernel<EPI, TPG>), dim3(grid), dim3(kRowsThreads), (size_t)rows_lds(TPG, a.cols), s, a, ntg);
}

template <int EPI>
static void launch_rows_epi(int tpg, const MmArgs &a, int ntg, unsigned grid, hipStream_t s) {
    switch (tpg) {
        case 2: launch_rows_one<EPI, 2>(a, ntg, grid, s); break;
        case 4: launch_rows_one<EPI, 4>(a, ntg, grid, s); break;
        case 8: launch_rows_one<EPI, 8>(a, ntg, grid, s); break;
        default: launch_rows_one<EPI, 16>(a, ntg, grid, s); break;
    }
}

// The small-batch kernel when it takes the product: Q8, a plain epilogue,
// at most kRowsMaxT tokens, or up to kRowsWideT when the product is small
// enough (rows·tokens up to kRowsWideWork: measured on MI355X, the 64 x 64
// tiles then cover few CUs and take longer, as for a short prompt's Wo;
// past it the tiles win, as for its QKV), and the staged inputs within LDS.
// Tokens per workgroup: halved (down to 2) while the workgroups still fit
// one round of about 1024 (four a CU).
constexpr int kRowsWideT = 64;
constexpr int64_t kRowsWideWork = 196608;
static bool launch_rows(int fmt, int epi, const MmArgs &a, hipStream_t s) {
    if (fmt != kFmtQ8 || (epi != kEpStore && epi != kEpAdd && epi != kEpAddCanon)) return false;
    if (a.tokens > kRowsMaxT && (a.tokens > kRowsWideT || (int64_t)a.rows * a.tokens > kRowsWideWork)) return false;
    const int64_t nrt = (a.rows + kRowsPerWg - 1) / kRowsPerWg;
    int tpg = kRowsMaxT;
    while (tpg > 2 && (tpg >= 2 * a.tokens || nrt * ((a.tokens + tpg / 2 - 1) / (tpg / 2)) <= 1024)) tpg >>= 1;
    if (rows_lds(tpg, a.cols) > 160 * 1024) return false;
    const int ntg = (a.tokens + tpg - 1) / tpg;
    const int64_t grid = ((nrt * ntg + 7) / 8) * 8;
    if (grid > INT32_MAX) return false;
    switch (epi) {
        case kEpStore: launch_rows_epi<kEpStore>(tpg, a, ntg, (unsigned)grid, s); break;
        case kEpAdd: launch_rows_epi<kEpAdd>(tpg, a, ntg, (unsigned)grid, s); break;
        default: launch_rows_epi<kEpAddCanon>(tpg, a, ntg, (unsigned)grid, s); break;
    }
    return true;
}

template <int FMT, int EPI>
static void launch_mm_one(const MmArgs &a, unsigned grid, hipStream_t s) {
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute((const void *)mm_kernel<FMT, EPI>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)(2 * sizeof(MmStage)));
    });
    RK_LAUNCH((mm_kernel<FMT, EPI>), dim3(grid), dim3(kMmThreads), 2 * sizeof(MmStage), s, a);
}

template <int FMT>
static bool launch_mm_epi(int epi, const MmArgs &a, unsigned grid, hipStream_t s) {
    switch (epi) {
        case kEpStore: launch_mm_one<FMT, kEpStore>(a, grid, s); return true;
        case kEpAdd: launch_mm_one<FMT, kEpAdd>(a, grid, s); return true;
        case kEpAddCanon: launch_mm_one<FMT, kEpAddCanon>(a, grid, s); return true;
        case kEpQKV: launch_mm_one<FMT, kEpQKV>(a, grid, s); return true;
        case kEpSilu: launch_mm_one<FMT, kEpSilu>(a, grid, s); return true;
    }
    return false;
}

bool launch_mm(int fmt, int epi, const MmArgs &a, hipStream_t s) {
    if (a.tokens <= 0 || a.rows <= 0) return true;
    if (a.cols < 32 || a.cols % 32 != 0) return false;
    if (epi == kEpSilu && (a.rows % 32 != 0 || a.nseg != 2)) return false;
    if (epi == kEpQKV && (a.hs % 2 != 0 || a.qdim % 2 != 0 || a.kvdim % 2 != 0 || a.row_base % 2 != 0)) return false;
    if (launch_rows(fmt, epi, a, s)) return true;
    const int ntr = epi == kEpSilu ? a.rows / 32 : (a.rows + kMmRows - 1) / kMmRows;
    const int ntt = (a.tokens + kMmToks - 1) / kMmToks;
    const int64_t total = (int64_t)ntr * ntt;
    const int64_t grid = ((total + 7) / 8) * 8;
    if (grid > INT32_MAX) return false;
    if (fmt == kFmtQ8) return launch_mm_epi<kFmtQ8>(epi, a, (unsigned)grid, s);
    if (fmt == kFmtQ4) return launch_mm_epi<kFmtQ4>(epi, a, (unsigned)grid, s);
    return false;
}

}  // namespace rk
