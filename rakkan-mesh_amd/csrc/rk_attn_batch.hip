// rk_attn_batch.hip — attention for a batch of consecutive positions (a
// prompt's prefill), a group of tokens per workgroup. Token z of the batch
// sits at position pos0 + z and attends to positions 0..pos0+z in exactly
// the order of one decode step (internal/llm/model.go:575-591):
//
//   scores  s_t = float32(Dot32(q, k_t)·invSqrt)  (element i into running sum
//           i mod 32, e_j = (s_j+s_j+8)+(s_j+16+s_j+24), the 8-tree)
//   softmax Go max, e_t = Exp32(s_t - max), one sequential sum, inv =
//           Recip32(sum), a_t = e_t·inv
//   values  out_i = Σ_t a_t·v_t,i in t order from +0
//
// What a group changes is only who loads what: a key tile serves the
// group's sixteen queries, a value tile the group's sixteen weight rows, and
// a workgroup runs sixteen tokens' sequential sums side by side (one per
// half-wave for the softmax, one per lane and element for the values, a
// lane holding the elements e, e+32, e+64, e+96 of its token).
#include <mutex>

#include "rk_dev.h"
#include "rk_fused.h"

namespace rk {

namespace {

constexpr int kGrpTok = 16;    // tokens per workgroup
constexpr int kGrpMaxT = 1024;  // positions a group's weights keep in LDS
constexpr int kScTile = 64;    // positions per scores workgroup
// The values workgroup's shape: SL 32-element slices of a head (SL = 4, or
// 1 for grids too small to fill the machine otherwise); its value tiles hold
// 128/SL positions (two a thread) of 32·SL elements.
#define RK_GV_SHAPE(SL)                                                                        \
    constexpr int kGvSlices = SL;                    /* slices per workgroup */                \
    constexpr int kGvElems = 32 * kGvSlices;         /* elements per workgroup */              \
    constexpr int kGvChunk = 128 / kGvSlices;        /* value positions per LDS tile */        \
    constexpr int kGvPitch = kGvChunk + 4;           /* floats per element row (odd count of 16-byte units) */
constexpr int kGvThreads = 512;         // eight waves, two tokens each
constexpr int kHs = 128;                // head size of the scores kernel

// acc[s] + Σ a[t]·v_s[t] for t < n in order, for the SL rows v_s = v +
// 32·s·kGvPitch (float32; each product rounded, then added), a and v in LDS
// (16-byte aligned). Independent chains (SL of them) keep the adds issuing;
// the next four positions' reads are issued before the current ones are
// summed.
template <int SL>
__device__ __forceinline__ void lds_dot_chain(const float *a, const float *v, int n, float (&acc)[SL]) {
    constexpr int kGvSlices = SL, kGvPitch = 128 / SL + 4;  // as RK_GV_SHAPE(SL)
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    const int nq = n >> 2;
    auto vq = [&](int s, int k) { return reinterpret_cast<const float4 *>(v + 32 * s * kGvPitch)[k]; };
    auto add4 = [&](const float4 &ca, const float4 (&cv)[kGvSlices]) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < kGvSlices; s++) acc[s] += ca.x * cv[s].x;
#pragma unroll
        for (int s = 0; s < kGvSlices; s++) acc[s] += ca.y * cv[s].y;
#pragma unroll
        for (int s = 0; s < kGvSlices; s++) acc[s] += ca.z * cv[s].z;
#pragma unroll
        for (int s = 0; s < kGvSlices; s++) acc[s] += ca.w * cv[s].w;
    };
    if (nq > 0) {
        float4 ca = a4[0], cv[kGvSlices];
#pragma unroll
        for (int s = 0; s < kGvSlices; s++) cv[s] = vq(s, 0);
        for (int k = 1; k < nq; k++) {
            float4 na = a4[k], nv[kGvSlices];
#pragma unroll
            for (int s = 0; s < kGvSlices; s++) nv[s] = vq(s, k);
            __builtin_amdgcn_sched_barrier(0);
            add4(ca, cv);
            __builtin_amdgcn_sched_barrier(0);
            ca = na;
#pragma unroll
            for (int s = 0; s < kGvSlices; s++) cv[s] = nv[s];
        }
        add4(ca, cv);
    }
    for (int t = nq << 2; t < n; t++)
#pragma unroll
        for (int s = 0; s < kGvSlices; s++) acc[s] += a[t] * v[32 * s * kGvPitch + t];
}

}  // namespace

// Scores of kScTile positions for the group's tokens, one head (size 128).
// Thread (position p = tid/4, part = tid%4) keeps its key's elements
// 8·part..8·part+7 of each 32-element step in registers, i.e. running sums
// j = 8·part..+7 of Dot32, and combines them with the other three parts by
// DPP, as the decode kernel does.
__global__ __launch_bounds__(256) void att_scores_group_kernel(const float *q, const float *keys, float *att,
                                                               int32_t att_stride, AttBatch bt, int kv_mul,
                                                               int kv_dim, float inv_sqrt) {
    __shared__ __align__(16) float sq[kGrpTok][kHs];
    const int h = blockIdx.x, g = h / kv_mul;
    const int t0 = blockIdx.y * kScTile;
    const int z0 = blockIdx.z * kGrpTok;
    const int nz = min(kGrpTok, bt.tokens - z0);
    const int tmax = bt.pos0 + z0 + nz;  // positions the group's last token sees
    if (t0 >= tmax) return;
    const int part = threadIdx.x & 3;
    const int t = t0 + (threadIdx.x >> 2);
    for (int i = threadIdx.x; i < kGrpTok * kHs / 4; i += 256) {
        const int zl = i / (kHs / 4), e4 = i % (kHs / 4);
        reinterpret_cast<float4 *>(&sq[zl][0])[e4] = reinterpret_cast<const float4 *>(
            q + (int64_t)(z0 + min(zl, nz - 1)) * bt.q_stride + (int64_t)h * kHs)[e4];
    }
    const float *kt = keys + (int64_t)min(t, tmax - 1) * kv_dim + (int64_t)g * kHs;
    float4 k0[kHs / 32], k1[kHs / 32];
#pragma unroll
    for (int st = 0; st < kHs / 32; st++) {
        k0[st] = *reinterpret_cast<const float4 *>(kt + 32 * st + 8 * part);
        k1[st] = *reinterpret_cast<const float4 *>(kt + 32 * st + 8 * part + 4);
    }
    __syncthreads();
    for (int zl = 0; zl < nz; zl++) {
        float s[8];
#pragma unroll
        for (int k = 0; k < 8; k++) s[k] = 0.0f;
#pragma unroll
        for (int st = 0; st < kHs / 32; st++) {
            const float4 q0 = *reinterpret_cast<const float4 *>(&sq[zl][32 * st + 8 * part]);
            const float4 q1 = *reinterpret_cast<const float4 *>(&sq[zl][32 * st + 8 * part + 4]);
            s[0] += q0.x * k0[st].x;
            s[1] += q0.y * k0[st].y;
            s[2] += q0.z * k0[st].z;
            s[3] += q0.w * k0[st].w;
            s[4] += q1.x * k1[st].x;
            s[5] += q1.y * k1[st].y;
            s[6] += q1.z * k1[st].z;
            s[7] += q1.w * k1[st].w;
        }
        float e[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float u = s[k] + dppf_x1(s[k]);  // part 0: s_j + s_j+8; part 2: s_j+16 + s_j+24
            e[k] = u + dppf_x2(u);                 // part 0: e_j
        }
        const float dot = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
        const int z = z0 + zl;
        if (part == 0 && t < bt.pos0 + z + 1)
            att[(int64_t)z * bt.att_stride + (int64_t)h * att_stride + t] = dot * inv_sqrt;
    }
}

// Softmax and weighted values of up to SL 32-element slices of one head
// (elements e0 .. e0+32·SL-1) for the group's tokens. Half-wave zl (lanes
// 32·(zl&1).. of wave zl/2) owns token z0 + zl: its softmax over its
// positions, once, then the sums of elements e0 + 32·s + lane%32.
template <int SL>
__global__ __launch_bounds__(kGvThreads) void att_values_group_kernel(const float *att, int32_t att_stride,
                                                                      const float *vals, float *out, AttBatch bt,
                                                                      int kv_mul, int hs, int kv_dim, int apitch,
                                                                      int8_t *qx, float *xs, int32_t *xsum) {
    RK_GV_SHAPE(SL)
    extern __shared__ __align__(16) float smem[];
    __shared__ float s_inv[kGrpTok];
    __shared__ __align__(16) float s_out[kGrpTok][kGvElems];
    float *sa = smem;                         // [kGrpTok][apitch] weights a_t
    float *vt = smem + kGrpTok * apitch;      // [2][kGvElems][kGvPitch] value tiles, transposed
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x, g = h / kv_mul;
    const int e0 = blockIdx.y * kGvElems;
    const int ns = min(kGvSlices, (hs - e0) >> 5);  // slices of the head here
    // the last token groups (the most positions) are dispatched first, so
    // the short ones fill the machine's last round
    const int z0 = (int)(gridDim.z - 1 - blockIdx.z) * kGrpTok;
    const int nz = min(kGrpTok, bt.tokens - z0);
    const int zl = 2 * wave + (lane >> 5), l32 = lane & 31;
    const int zc = min(zl, nz - 1);      // halves past the batch repeat its last token, unstored
    const int Tz = bt.pos0 + z0 + zc + 1;
    const int tmax = bt.pos0 + z0 + nz;
    float *az = sa + zl * apitch;

    // ---- the value tiles' loads: thread (elements e0 + 4·fq.., positions
    // 2·pq, 2·pq+1 of the chunk); positions past tmax and elements past the
    // head clamped, never summed or stored
    const int fq = tid % (kGvElems / 4), pq = tid / (kGvElems / 4);
    const float *vbase = vals + (int64_t)g * hs + min(e0 + 4 * fq, hs - 4);
    float4 v0, v1;
    auto load_tile = [&](int c0) {
        v0 = *reinterpret_cast<const float4 *>(vbase + (int64_t)min(c0 + 2 * pq, tmax - 1) * kv_dim);
        v1 = *reinterpret_cast<const float4 *>(vbase + (int64_t)min(c0 + 2 * pq + 1, tmax - 1) * kv_dim);
    };
    auto store_tile = [&](float *tile) {
        float *d = tile + (4 * fq) * kGvPitch + 2 * pq;
        *reinterpret_cast<float2 *>(d) = make_float2(v0.x, v1.x);
        *reinterpret_cast<float2 *>(d + kGvPitch) = make_float2(v0.y, v1.y);
        *reinterpret_cast<float2 *>(d + 2 * kGvPitch) = make_float2(v0.z, v1.z);
        *reinterpret_cast<float2 *>(d + 3 * kGvPitch) = make_float2(v0.w, v1.w);
    };
    load_tile(0);  // in flight during the softmax

    // ---- softmax of each half's token ----
    const float *row = att + (int64_t)(z0 + zc) * bt.att_stride + (int64_t)h * att_stride;
    float m = row[0];
    for (int t = l32; t < Tz; t += 32) {
        const float v = row[t];
        az[t] = v;
        m = gomax(m, v);
    }
    m = half_gomax(m);
    for (int t = l32; t < Tz; t += 32) az[t] = exp32(az[t] - m);
    __syncthreads();
    if (l32 == 0) s_inv[zl] = recip32(lds_chain_sum(az, Tz, 0.0f));
    __syncthreads();
    const float inv = s_inv[zl];
    for (int t = l32; t < Tz; t += 32) az[t] = az[t] * inv;

    // ---- values: tiles of kGvChunk positions, double-buffered ----
    store_tile(vt);
    __syncthreads();
    float acc[kGvSlices] = {};
    int buf = 0;
    for (int c0 = 0; c0 < tmax; c0 += kGvChunk, buf ^= 1) {
        load_tile(c0 + kGvChunk);  // the next tile, in flight during the sums
        const float *tile = vt + buf * (kGvElems * kGvPitch);
        const int n = max(0, min(kGvChunk, Tz - c0));
        lds_dot_chain<SL>(az + c0, tile + l32 * kGvPitch, n, acc);
        // the other buffer was last read two tiles ago, before the barrier
        // that ended that iteration
        store_tile(vt + (buf ^ 1) * (kGvElems * kGvPitch));
        __syncthreads();
    }

    const bool live = zl < nz;
    const int64_t base = (int64_t)(z0 + zl) * bt.out_stride + (int64_t)h * hs + e0;
#pragma unroll
    for (int s = 0; s < kGvSlices; s++)
        if (live && s < ns) out[base + 32 * s + l32] = acc[s];
    if (qx) {
        // each slice is one Q8_0 block of each token's next input (hs is a
        // multiple of 32): lanes 8·s.. 8·s+7 of the half take slice s, four
        // values each (every lane calls the quantizer)
#pragma unroll
        for (int s = 0; s < kGvSlices; s++) s_out[zl][32 * s + l32] = acc[s];
        __syncthreads();
        const int sb = min(l32 >> 3, kGvSlices - 1), q = l32 & 7;
        const float4 v4 = reinterpret_cast<const float4 *>(&s_out[zl][32 * sb])[q];
        float d;
        int cs;
        const uint32_t pk = quantize_group(v4.x, v4.y, v4.z, v4.w, d, cs);
        const int64_t bb = base + 32 * sb;
        if (live && (l32 >> 3) < ns) {
            reinterpret_cast<uint32_t *>(qx + bb)[q] = pk;
            if (q == 0) {
                xs[bb >> 5] = d;
                xsum[bb >> 5] = cs;
            }
        }
    }
}

bool att_group_fits(const AttBatch &bt, int hs, int kv_dim) {
    // (consecutive positions of one sequence only)
    return !bt.pos && bt.pos0 + bt.tokens <= kGrpMaxT && hs % 32 == 0 && kv_dim % 4 == 0;
}

void launch_att_scores_group(const float *q, const float *keys, float *att, int32_t att_stride, const AttBatch &bt,
                             int heads, int kv_heads, int kv_dim, float inv_sqrt, hipStream_t s) {
    const int npos = bt.pos0 + bt.tokens;
    const dim3 grid(heads, (npos + kScTile - 1) / kScTile, (bt.tokens + kGrpTok - 1) / kGrpTok);
    RK_LAUNCH(att_scores_group_kernel, grid, dim3(256), 0, s, q, keys, att, att_stride, bt, heads / kv_heads, kv_dim,
              inv_sqrt);
}

template <int SL>
static void launch_values_sl(const float *att, int32_t att_stride, const float *vals, float *out, const AttBatch &bt,
                             int heads, int kv_heads, int hs, int kv_dim, int8_t *qx, float *xs, int32_t *xsum,
                             hipStream_t s) {
    RK_GV_SHAPE(SL)
    static std::once_flag once;
    std::call_once(once, [] {
        (void)hipFuncSetAttribute((const void *)att_values_group_kernel<SL>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kMaxLdsBytes - 12288));
    });
    const int tmax = bt.pos0 + bt.tokens;
    const int apitch = ((tmax + 3) & ~3) + 4;
    const size_t lds = ((size_t)kGrpTok * apitch + 2 * kGvElems * kGvPitch) * 4;
    const dim3 grid(heads, (hs + kGvElems - 1) / kGvElems, (bt.tokens + kGrpTok - 1) / kGrpTok);
    RK_LAUNCH(att_values_group_kernel<SL>, grid, dim3(kGvThreads), lds, s, att, att_stride, vals, out, bt,
              heads / kv_heads, hs, kv_dim, apitch, qx, xs, xsum);
}

void launch_att_values_group(const float *att, int32_t att_stride, const float *vals, float *out, const AttBatch &bt,
                             int heads, int kv_heads, int hs, int kv_dim, int8_t *qx, float *xs, int32_t *xsum,
                             hipStream_t s, int cu) {
    // four slices a workgroup (the softmax once per head and token group)
    // unless that leaves fewer workgroups than the device has CUs (a short
    // batch; cu 0: the MI355X's 256): then one slice a workgroup, four
    // times the workgroups
    const int64_t wgs4 = (int64_t)heads * ((hs + 127) / 128) * ((bt.tokens + kGrpTok - 1) / kGrpTok);
    if (wgs4 >= (cu > 0 ? cu : 256))
        launch_values_sl<4>(att, att_stride, vals, out, bt, heads, kv_heads, hs, kv_dim, qx, xs, xsum, s);
    else
        launch_values_sl<1>(att, att_stride, vals, out, bt, heads, kv_heads, hs, kv_dim, qx, xs, xsum, s);
}

}  // namespace rk
