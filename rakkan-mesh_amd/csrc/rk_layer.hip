// rk_layer.hip — the llama-family layer operations for gfx950, each doing
// what internal/llm's Stage.Forward does on the CPU in the same order of
// float32 operations (internal/llm/model.go:522-657), so results are the
// CPU's bits:
//   RMSNorm   ss = Dot32(x,x)·recipN + eps, out = w·(Rsqrt32(ss)·x)
//   RoPE      adjacent pairs: (v0·c − v1·s, v0·s + v1·c)
//   attention score = Dot32(q_h, k_t)·invSqrt; softmax (Go max, Exp32,
//             one sequential sum, ·Recip32(sum)); out += a_t·v_t in t order
//   SiLU·mul  a = (a·Recip32(1 + Exp32(−a)))·b
//   residual  x += y (canonical NaN when asked)
// Dot32 is the 32-sum order of internal/num/matvec.go:32-66: element i into
// sum i mod 32, then e_j = (s_j + s_j+8) + (s_j+16 + s_j+24), then the
// ((e0+e1)+(e2+e3))+((e4+e5)+(e6+e7)) tree.
#include "rk_fmath.h"
#include "rk_layer.h"

namespace rk {

// Dot32 by the 32 lanes of a half-wave (lanes 0-31 or 32-63, `hl` = lane in
// the half); the result is valid in the half's lane 0. Every lane of the
// wave must call it (cross-lane moves).
__device__ __forceinline__ float dot32_half(const float *a, const float *b, int n, int hl, bool valid) {
    float s = 0.0f;
    if (valid)
        for (int i = hl; i < n; i += 32) s += a[i] * b[i];
    const float s8 = __shfl_down(s, 8, 32), s16 = __shfl_down(s, 16, 32), s24 = __shfl_down(s, 24, 32);
    const float e = (s + s8) + (s16 + s24);  // lanes 0..7 of the half
    const float p = e + __shfl_down(e, 1, 32);
    const float q = p + __shfl_down(p, 2, 32);
    return q + __shfl_down(q, 4, 32);
}

// Dot32 over a whole wave; the result is returned in every lane.
__device__ __forceinline__ float dot32_wave(const float *a, const float *b, int n) {
    const int lane = threadIdx.x & 63;
    const float r = dot32_half(a, b, n, lane, lane < 32);
    return __shfl(r, 0);
}

// ---------------------------------------------------------------------------
// RMSNorm of segments (internal/gpu/kernels.go:355-392, internal/llm/model.go:
// 632-638): one wave per segment, `stride` floats apart; out may be in.
__global__ __launch_bounds__(64) void rmsnorm_kernel(const float *in, float *out, const float *w, int n, int64_t stride,
                                                     float recip_n, float eps) {
    const float *x = in + blockIdx.x * stride;
    float *o = out + blockIdx.x * stride;
    const float dot = dot32_wave(x, x, n);
    const float ss = (dot * recip_n) + eps;
    const float r = rsqrt32(ss);
    for (int i = threadIdx.x; i < n; i += 64) o[i] = w[i] * (r * x[i]);
}

void launch_rmsnorm(const float *in, float *out, const float *w, int n, int segs, int64_t stride, float recip_n,
                    float eps, hipStream_t s) {
    if (segs <= 0 || n <= 0) return;
    RK_LAUNCH(rmsnorm_kernel, dim3(segs), dim3(64), 0, s, in, out, w, n, stride, recip_n, eps);
}

// out += v (internal/gpu/kernels.go:394-404).
__global__ void addvec_kernel(float *out, const float *v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = out[i] + v[i];
}

void launch_addvec(float *out, const float *v, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    RK_LAUNCH(addvec_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, v, n);
}

// Rotary embedding of adjacent pairs (internal/gpu/kernels.go:406-427,
// internal/llm/model.go:563-572): pair p of q, and of k while 2p < kvDim.
__global__ void rope_kernel(float *q, float *k, int pairs, int kv_dim, int hs, const float *cos_row,
                            const float *sin_row) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= pairs) return;
    const int i = 2 * p;
    const int pi = (i % hs) / 2;
    const float co = cos_row[pi], si = sin_row[pi];
    {
        const float v0 = q[i], v1 = q[i + 1];
        q[i] = (v0 * co) - (v1 * si);
        q[i + 1] = (v0 * si) + (v1 * co);
    }
    if (i < kv_dim) {
        const float v0 = k[i], v1 = k[i + 1];
        k[i] = (v0 * co) - (v1 * si);
        k[i + 1] = (v0 * si) + (v1 * co);
    }
}

void launch_rope(float *q, float *k, int q_dim, int kv_dim, int hs, const float *cos_row, const float *sin_row,
                 hipStream_t s) {
    const int pairs = q_dim / 2;
    if (pairs <= 0) return;
    RK_LAUNCH(rope_kernel, dim3((pairs + 255) / 256), dim3(256), 0, s, q, k, pairs, kv_dim, hs, cos_row,
                       sin_row);
}

// Word copy (internal/gpu/kernels.go:429-437).
__global__ void copy_kernel(const uint32_t *src, uint32_t *dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

void launch_copy(const void *src, void *dst, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    RK_LAUNCH(copy_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const uint32_t *)src,
                       (uint32_t *)dst, n);
}

// x += y, canonical NaN if asked (internal/gpu/kernels.go:552-563).
__global__ void residual_kernel(float *x, const float *y, int64_t n, int canon) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i] + y[i];
    x[i] = canon ? canonical(v) : v;
}

void launch_residual(float *x, const float *y, int64_t n, bool canon, hipStream_t s) {
    if (n <= 0) return;
    RK_LAUNCH(residual_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n, canon ? 1 : 0);
}

// a = silu(a)·b (internal/gpu/kernels.go:565-577, internal/llm/model.go:657).
__global__ void silumul_kernel(float *a, const float *b, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = a[i];
    const float sl = v * recip32(1.0f + exp32(-v));
    a[i] = sl * b[i];
}

void launch_silumul(float *a, const float *b, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    RK_LAUNCH(silumul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, b, n);
}

// ---------------------------------------------------------------------------
// Attention for one position (internal/gpu/kernels.go:439-550, internal/llm/
// model.go:575-591), one workgroup per query head: scores into att (heads
// rows, att_stride apart), softmax in place, then the weighted values.
constexpr int kAttThreads = 256;

__global__ __launch_bounds__(kAttThreads) void attention_kernel(const float *q, const float *keys, const float *vals,
                                                                float *att, int64_t att_stride, float *out, int T,
                                                                int kv_mul, int hs, int kv_dim, float inv_sqrt) {
    __shared__ float red[kAttThreads];
    __shared__ float bcast;
    const int h = blockIdx.x;
    const int g = h / kv_mul;
    const int tid = threadIdx.x;
    const float *qh = q + (int64_t)h * hs;
    float *ah = att + (int64_t)h * att_stride;

    // Scores: a half-wave per position, eight positions per pass.
    const int half = tid >> 5, hl = tid & 31;
    for (int tb = 0; tb < T; tb += kAttThreads / 32) {
        const int t = tb + half;
        const bool valid = t < T;
        const float *kt = keys + (int64_t)(valid ? t : 0) * kv_dim + (int64_t)g * hs;
        const float d = dot32_half(qh, kt, hs, hl, valid);
        if (valid && hl == 0) ah[t] = d * inv_sqrt;
    }
    __syncthreads();

    // Maximum with Go's max (exact in any order).
    float m = ah[0];
    for (int t = tid; t < T; t += kAttThreads) m = gomax(m, ah[t]);
    red[tid] = m;
    __syncthreads();
    if (tid == 0) {
        float mm = red[0];
        for (int i = 1; i < kAttThreads; i++) mm = gomax(mm, red[i]);
        bcast = mm;
    }
    __syncthreads();
    const float mx = bcast;
    for (int t = tid; t < T; t += kAttThreads) ah[t] = exp32(ah[t] - mx);
    __syncthreads();
    // One sequential sum, in position order.
    if (tid == 0) {
        float sum = 0.0f;
        int t = 0;
        for (; t + 8 <= T; t += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = ah[t + j];
#pragma unroll
            for (int j = 0; j < 8; j++) sum += v[j];
        }
        for (; t < T; t++) sum += ah[t];
        bcast = recip32(sum);
    }
    __syncthreads();
    const float inv = bcast;
    for (int t = tid; t < T; t += kAttThreads) ah[t] = ah[t] * inv;
    __syncthreads();

    // Weighted values, each element summed over positions in order from +0.
    for (int i = tid; i < hs; i += kAttThreads) {
        const float *v = vals + (int64_t)g * hs + i;
        float acc = 0.0f;
        int t = 0;
        for (; t + 4 <= T; t += 4) {
            const float a0 = ah[t], a1 = ah[t + 1], a2 = ah[t + 2], a3 = ah[t + 3];
            const float v0 = v[(int64_t)t * kv_dim], v1 = v[(int64_t)(t + 1) * kv_dim];
            const float v2 = v[(int64_t)(t + 2) * kv_dim], v3 = v[(int64_t)(t + 3) * kv_dim];
            acc += a0 * v0;
            acc += a1 * v1;
            acc += a2 * v2;
            acc += a3 * v3;
        }
        for (; t < T; t++) acc += ah[t] * v[(int64_t)t * kv_dim];
        out[(int64_t)h * hs + i] = acc;
    }
}

void launch_attention(const float *q, const float *keys, const float *vals, float *att, int64_t att_stride, float *out,
                      int positions, int heads, int kv_heads, int hs, int kv_dim, float inv_sqrt, hipStream_t s) {
    if (positions <= 0 || heads <= 0) return;
    RK_LAUNCH(attention_kernel, dim3(heads), dim3(kAttThreads), 0, s, q, keys, vals, att, att_stride, out,
                       positions, heads / kv_heads, hs, kv_dim, inv_sqrt);
}

// ---------------------------------------------------------------------------
// Embedding row (internal/llm/model.go:216-231 Row, :660-664 Embed):
// x_i = float32(q_i · scale_i/32) for Q8_0, DequantQ8's expansion for Q4_0.
__global__ void embed_kernel(const uint8_t *w, const float *scales, int kind, const int32_t *token, int dim,
                             float *x) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    const int64_t tok = *token;
    const int nb = dim >> 5;
    const float d = scales[tok * nb + (i >> 5)];
    if (kind == 0) {
        const int8_t *row = reinterpret_cast<const int8_t *>(w) + tok * dim;
        x[i] = (float)row[i] * d;
    } else {
        const uint8_t *row = w + tok * (dim / 2);
        const int b = i >> 5, j = i & 31;
        const uint8_t v = row[b * 16 + (j & 15)];
        const int c = (j < 16 ? (v & 15) : (v >> 4)) - 8;
        x[i] = (float)c * d;
    }
}

void launch_embed(const uint8_t *w, const float *scales, bool q4, const int32_t *token, int dim, float *x,
                  hipStream_t s) {
    RK_LAUNCH(embed_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, w, scales, q4 ? 1 : 0, token, dim, x);
}

// Greedy argmax (internal/llm/sample.go:45-53): the first index holding the
// largest value, `>` comparisons (NaNs never win; a NaN at 0 stays).
__global__ __launch_bounds__(1024) void argmax_kernel(const float *v, int64_t n, int32_t *out) {
    __shared__ float bv[1024];
    __shared__ int64_t bi[1024];
    const int tid = threadIdx.x;
    float best = -__builtin_inff();
    int64_t idx = -1;
    for (int64_t i = tid; i < n; i += 1024) {
        const float x = v[i];
        if (idx < 0 ? (x == x) : (x > best)) {
            best = x;
            idx = i;
        }
    }
    bv[tid] = best;
    bi[tid] = idx;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
        if (tid < w) {
            const float ob = bv[tid + w];
            const int64_t oi = bi[tid + w];
            if (oi >= 0 && (bi[tid] < 0 || ob > bv[tid] || (ob == bv[tid] && oi < bi[tid]))) {
                bv[tid] = ob;
                bi[tid] = oi;
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        const float v0 = v[0];
        *out = (v0 != v0 || bi[0] < 0) ? 0 : (int32_t)bi[0];
    }
}

void launch_argmax(const float *v, int64_t n, int32_t *out, hipStream_t s) {
    RK_LAUNCH(argmax_kernel, dim3(1), dim3(1024), 0, s, v, n, out);
}

}  // namespace rk
