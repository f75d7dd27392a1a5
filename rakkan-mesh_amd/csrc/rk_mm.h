// rk_mm.h — batched quantized products (prompt prefill) on int8 MFMA: the
// same per-(token, row) results as the batch-1 kernels, for many tokens at
// once.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rk_fused.h"
#include "rk_kernels.h"

namespace rk {

// One batched product: rows of up to three matrices (concatenated; for
// kEpSilu seg[0] = W1 and seg[1] = W3, paired row by row) times `tokens`
// quantized inputs.
struct MmArgs {
    MatSeg seg[3];     // kEpStore: seg[i].out is [tokens][seg[i].rows]
    int32_t nseg;
    int32_t cols;      // input width (multiple of 32)
    int32_t rows;      // output rows (kEpSilu: rows of W1)
    int32_t tokens;
    const int8_t *qx;  // [tokens][cols] codes
    const float *xs;   // [tokens][cols/32] block scales
    // epilogue
    const float *bias;           // per output row (kEpStore, kEpQKV), or null
    float *x;                    // kEpAdd / kEpAddCanon: residual [tokens][ldx]
    int32_t ldx;
    int32_t row_base;            // kEpQKV: logical q/k/v row (and bias index) of row 0
    int32_t pos0;                // kEpQKV: position of token 0
    const int32_t *seq_pos;      // kEpQKV, independent sequences: token t at seq_pos[t] (device), not pos0 + t,
    int64_t cache_stride;        //   in caches cache_stride floats after token t-1's
    int32_t hs, qdim, kvdim;     // kEpQKV: head size, q rows, k rows (= v rows)
    const float *cos_t, *sin_t;  // kEpQKV: rotary table [ctx][hs/2]
    float *q;                    // kEpQKV: [tokens][qdim]
    float *kcache, *vcache;      // kEpQKV: [ctx][kvdim]
    int8_t *qx_out;              // kEpSilu: h quantized, [tokens][rows] codes
    float *xs_out;               //          [tokens][rows/32] scales
    int32_t *xsum_out;           //          [tokens][rows/32] code sums
};

// Enqueues the product; false when the epilogue or shape is not supported
// (kEpLogits; kEpSilu with rows not a multiple of 32).
bool launch_mm(int fmt, int epi, const MmArgs &a, hipStream_t s);

}  // namespace rk
