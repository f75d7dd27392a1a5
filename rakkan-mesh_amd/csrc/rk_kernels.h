// rk_kernels.h — host-side launchers of the gfx950 kernels (internal to
// librkhip; the C-ABI is include/rk.h).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rk {

// Timing of the next launch: when set (by the library's profiler), a launch
// hands these events to the dispatch itself, so the command processor stamps
// the kernel's own start and end (hipExtLaunchKernelGGL).
struct LaunchEvents {
    hipEvent_t start, stop;
};
extern thread_local LaunchEvents *g_launch_events;

#define RK_LAUNCH(kernel, grid, block, shmem, stream, ...)                                                  \
    do {                                                                                                    \
        if (::rk::g_launch_events)                                                                          \
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, ::rk::g_launch_events->start,        \
                                  ::rk::g_launch_events->stop, 0, __VA_ARGS__);                             \
        else                                                                                                \
            hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                            \
    } while (0)

// One matrix of a multi-matrix product: rows of packed codes (`row_bytes`
// apart) and [rows][cols/32] float scales, results to out[0..rows).
struct MatSeg {
    const uint8_t *w;
    const float *ws;
    float *out;
    int64_t rows;
};

constexpr int kMaxSegs = 4;

// What a product does with a row's result: store it, or add it to the
// output's value (a residual connection), optionally canonicalising NaNs.
enum : int32_t { kEpiStore = 0, kEpiAdd = 1, kEpiAddCanonical = 2 };

struct MatvecArgs {
    MatSeg seg[kMaxSegs];
    int32_t nseg;
    int32_t cols;
    int64_t total_rows;
    int64_t per_wave;    // rows of each wavefront (set by the launcher)
    int32_t epilogue;    // kEpi*
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
