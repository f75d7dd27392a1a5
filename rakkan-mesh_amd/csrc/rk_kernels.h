// rk_kernels.h — host-side launchers of the gfx950 kernels (internal to
// librkhip; the C-ABI is include/rk.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rk {

// One matrix of a multi-matrix product: rows of packed codes (`row_bytes`
// apart) and [rows][cols/32] float scales, results to out[0..rows).
struct MatSeg {
    const uint8_t *w;
    const float *ws;
    float *out;
    int64_t rows;
};

constexpr int kMaxSegs = 4;

struct MatvecArgs {
    MatSeg seg[kMaxSegs];
    int32_t nseg;
    int32_t cols;
    int64_t total_rows;
    int64_t per_wave;    // rows of each wavefront (set by the launcher)
    const int8_t *qx;    // quantized input, cols bytes
    const float *xs;     // its block scales, cols/32
    const int32_t *xsum; // per-block sums of qx (Q4's nibble offset)
};

// Activation quantize (internal/num/quant.go:34-53): x[n] -> qx[n], xs[n/32],
// xsum[n/32] (sum of the block's codes).
void launch_quantize_acts(const float *x, int64_t n, int8_t *qx, float *xs, int32_t *xsum, hipStream_t s);

// Q8_0 / Q4_0 products of the quantized input with up to kMaxSegs matrices
// sharing cols (internal/num/quant.go:158-196). cu = compute units.
void launch_matvec_q8(const MatvecArgs &a, int cu, hipStream_t s);
void launch_matvec_q4(const MatvecArgs &a, int cu, hipStream_t s);

}  // namespace rk
