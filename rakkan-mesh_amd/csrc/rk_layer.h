// rk_layer.h — launchers of the layer kernels (rk_layer.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rk_kernels.h"

namespace rk {

void launch_rmsnorm(const float *in, float *out, const float *w, int n, int segs, int64_t stride, float recip_n,
                    float eps, hipStream_t s);
void launch_addvec(float *out, const float *v, int64_t n, hipStream_t s);
void launch_rope(float *q, float *k, int q_dim, int kv_dim, int hs, const float *cos_row, const float *sin_row,
                 hipStream_t s);
void launch_copy(const void *src, void *dst, int64_t n, hipStream_t s);
void launch_residual(float *x, const float *y, int64_t n, bool canon, hipStream_t s);
void launch_silumul(float *a, const float *b, int64_t n, hipStream_t s);
void launch_attention(const float *q, const float *keys, const float *vals, float *att, int64_t att_stride, float *out,
                      int positions, int heads, int kv_heads, int hs, int kv_dim, float inv_sqrt, hipStream_t s);
void launch_embed(const uint8_t *w, const float *scales, bool q4, const int32_t *token, int dim, float *x,
                  hipStream_t s);
void launch_argmax(const float *v, int64_t n, int32_t *out, hipStream_t s);

}  // namespace rk
