// rk_mx.h — DeepSeek-V4.1 block-scaled products (E4M3 and E2M1 weights
// with E8M0 scales) and their input quantization, for gfx950.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rk {

// internal/num/mx.go:185-203 QuantizeActFP8: n floats (a multiple of 32) to
// E4M3 codes and one power-of-two float32 scale per 32.
void launch_act_fp8(const float *x, int64_t n, uint8_t *codes, float *scales, hipStream_t s);

// The value of each of n E4M3 codes, unscaled, as float32 (the layout the
// reference's QuantizeFP8 leaves in the arena, internal/gpu/mx.go:146-172).
void launch_e4m3_values(const uint8_t *codes, int64_t n, float *out, hipStream_t s);

// mx.go:205-214 ActQuantInPlace and 268-290 FP4QuantInPlace of n floats
// (n a multiple of the block: 32, or 16 for E4M3 scales) in place.
void launch_act_quant_inplace(float *x, int64_t n, hipStream_t s);
void launch_fp4_quant_inplace(float *x, int64_t n, bool e4m3, hipStream_t s);

// The device layout of E2M1 scales: blocks of RT = 8 rows, a lane's rows
// together (byte (k·nb + b)·8 + r for row 8k + r, block b; zero past the
// last row). Its size, and the repacking of the reference layout
// [rows][cols/32] into it.
int64_t mx_fp4_scale_bytes(int64_t rows, int64_t cols);
void mx_fp4_pack_scales(const uint8_t *e8m0, int64_t rows, int64_t cols, uint8_t *dst);

// internal/num/mx.go:282-334 MatVecFP8 / MatVecFP4 of an input quantized by
// launch_act_fp8 (codes xc, scales xs): out[r] for rows rows; w E4M3
// [rows][cols] with E8M0 scales [ceil(rows/32)][cols/32] (fp4 = false), or
// E2M1 packed [rows][cols/2] with E8M0 scales in mx_fp4_pack_scales's
// layout (fp4 = true). raw leaves the sums in float32 instead of rounding
// them to bfloat16.
void launch_mx_matvec(bool fp4, const uint8_t *w, const uint8_t *ws, int64_t rows, int64_t cols, const uint8_t *xc,
                      const float *xs, float *out, bool raw, hipStream_t s);

// internal/gpu/dsbatch.go:142-172 ExpertMatVecs: E2M1 experts of per_expert
// rows stacked in w (experts of them; per_expert a multiple of 8); slot y
// (of slots) multiplies expert ids[y] (device memory; ids not below experts
// are skipped) by input y / div (codes xc + (y/div)·cols, scales
// xs + (y/div)·cols/32) into out + y·out_stride.
void launch_mx_experts(const uint8_t *w, const uint8_t *ws, int64_t experts, int64_t per_expert, int64_t cols,
                       const uint32_t *ids, int slots, int div, const uint8_t *xc, const float *xs, float *out,
                       int64_t out_stride, bool raw, hipStream_t s);

}  // namespace rk
