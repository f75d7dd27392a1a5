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
    bool launched;  // a launch in the scope recorded them
};
extern thread_local LaunchEvents *g_launch_events;

#define RK_LAUNCH(kernel, grid, block, shmem, stream, ...)                                                  \
    do {                                                                                                    \
        if (::rk::g_launch_events) {                                                                        \
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, ::rk::g_launch_events->start,        \
                                  ::rk::g_launch_events->stop, 0, __VA_ARGS__);                             \
            ::rk::g_launch_events->launched = true;                                                         \
        } else                                                                                              \
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

// Activation quantize (internal/num/quant.go:34-53): x[n] -> qx[n], xs[n/32],
// xsum[n/32] (sum of the block's codes).
void launch_quantize_acts(const float *x, int64_t n, int8_t *qx, float *xs, int32_t *xsum, hipStream_t s);

}  // namespace rk
