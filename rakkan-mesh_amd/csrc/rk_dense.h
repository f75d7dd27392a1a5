// rk_dense.h — launchers of the float32 / bfloat16 products (rk_dense.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rk {

// Elements per row of an uploaded float32 / bfloat16 matrix: cols rounded
// up to a multiple of 32, the padding zero.
int64_t dense_row_elems(int64_t cols);

// out[r] = Dot32(row r, x) for r < rows (internal/num/matvec.go:106-123
// MatVec32 / MatVecBF16): w holds rows of dense_row_elems(cols) float32
// (bf16 false) or bfloat16 (bf16 true) values; x and out device buffers.
void launch_dense_matvec(bool bf16, const void *w, int64_t rows, int64_t cols, const float *x, float *out,
                         hipStream_t s);

}  // namespace rk
