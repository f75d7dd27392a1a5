// rk_diag.hip — the floor a launch cannot go below on this device, measured
// on it: back-to-back launches of an empty kernel, and of a plain streaming
// read of a given number of bytes (16-byte coalesced loads, all of a
// thread's issued before any is used, nothing stored; the fastest of a few
// access shapes, load depths and workgroup sizes). A product that reads the same bytes
// cannot take less time per launch than the read; what it takes beyond it is
// its own arithmetic, waits and stores.
#include <algorithm>

#include "rk_runtime.h"

namespace rk {
namespace {

typedef int fv4i __attribute__((ext_vector_type(4)));


__global__ __launch_bounds__(64) void floor_empty_kernel(int *sink, int flag) {
    if (flag != 0 && threadIdx.x == 0) sink[0] = flag;  // the host passes 0
}

// Thread t of the grid reads pieces t, t + G, ..., t + (LOADS-1)G (G threads
// in the grid; pieces past the end re-read the last one). The XOR of what it
// read is stored only if it equals `flag`, which the host's fill never gives.
template <int LOADS>
__global__ __launch_bounds__(1024) void floor_read_kernel(const fv4i *p, int64_t n16, int *sink, int flag) {
    const int64_t g = (int64_t)gridDim.x * blockDim.x;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    fv4i v[LOADS];
#pragma unroll
    for (int k = 0; k < LOADS; k++) v[k] = __builtin_nontemporal_load(p + min(t + k * g, n16 - 1));
    int acc = 0;
#pragma unroll
    for (int k = 0; k < LOADS; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    if (acc == flag) sink[0] = acc;
}

// Wave w of the grid reads LOADS contiguous KiB, pieces 64·LOADS·w onwards
// (the access shape of a product's row), all issued before any is used.
template <int LOADS>
__global__ __launch_bounds__(1024) void floor_wave_kernel(const fv4i *p, int64_t n16, int *sink, int flag) {
    const int64_t w = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    fv4i v[LOADS];
#pragma unroll
    for (int k = 0; k < LOADS; k++) v[k] = __builtin_nontemporal_load(p + min((w * LOADS + k) * 64 + lane, n16 - 1));
    int acc = 0;
#pragma unroll
    for (int k = 0; k < LOADS; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    if (acc == flag) sink[0] = acc;
}

struct FloorShape {
    void (*fn)(const fv4i *, int64_t, int *, int);
    int loads, threads;
};
const FloorShape kFloorShapes[] = {
    {floor_read_kernel<4>, 4, 256},  {floor_read_kernel<8>, 8, 256},   {floor_read_kernel<8>, 8, 512},
    {floor_read_kernel<16>, 16, 256}, {floor_read_kernel<16>, 16, 512}, {floor_read_kernel<8>, 8, 1024},
    {floor_wave_kernel<4>, 4, 512},   {floor_wave_kernel<8>, 8, 512},   {floor_wave_kernel<14>, 14, 1024},
    {floor_wave_kernel<16>, 16, 512},
};

}  // namespace
}  // namespace rk

extern "C" int rk_device_launch_floor(rk_device *d, int64_t bytes, int32_t copies, int32_t launches,
                                      float *empty_us, float *read_us) {
    using namespace rk;
    if (!d || bytes < 16 || bytes % 16 || copies < 1 || launches < 1 || !empty_us || !read_us ||
        bytes > ((int64_t)1 << 36) / copies)
        return fail(d, RK_ERR_ARGS, "rk_device_launch_floor: bad arguments");
    Hold h(d->gate);
    if (d->capturing) return fail(d, RK_ERR_ARGS, "rk_device_launch_floor: the stream is recording a graph");
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    const hipStream_t s = d->stream;
    char *buf = nullptr;
    int *sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = RK_OK;
    auto run = [&]() -> int {
        HIP_TRY(d, hipMalloc(&buf, (size_t)bytes * copies), "launch floor buffer");
        HIP_TRY(d, hipMalloc(&sink, 64), "launch floor sink");
        // 0x01 bytes: every piece XORs to 0, never the flag
        HIP_TRY(d, hipMemsetAsync(buf, 1, (size_t)bytes * copies, s), "launch floor fill");
        HIP_TRY(d, hipEventCreate(&e0), "hipEventCreate");
        HIP_TRY(d, hipEventCreate(&e1), "hipEventCreate");
        const int64_t n16 = bytes / 16;
        const int flag = 0x7FFFFFFF;
        auto empties = [&](int n) {
            for (int i = 0; i < n; i++) hipLaunchKernelGGL(floor_empty_kernel, dim3(1), dim3(64), 0, s, sink, 0);
        };
        auto reads = [&](const FloorShape &f, int n) {
            const int64_t per = (int64_t)f.threads * f.loads;
            const unsigned grid = (unsigned)std::min<int64_t>((n16 + per - 1) / per, (int64_t)1 << 30);
            for (int i = 0; i < n; i++)
                hipLaunchKernelGGL(f.fn, dim3(grid), dim3(f.threads), 0, s,
                                   reinterpret_cast<const fv4i *>(buf + (size_t)(i % copies) * bytes), n16, sink, flag);
        };
        float ms = 0.0f;
        empties(8);
        HIP_TRY(d, hipEventRecord(e0, s), "hipEventRecord");
        empties(launches);
        HIP_TRY(d, hipEventRecord(e1, s), "hipEventRecord");
        HIP_TRY(d, hipEventSynchronize(e1), "hipEventSynchronize");
        HIP_TRY(d, hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
        *empty_us = ms * 1e3f / launches;
        float best = 0.0f;
        for (const FloorShape &f : kFloorShapes) {
            reads(f, copies);
            HIP_TRY(d, hipEventRecord(e0, s), "hipEventRecord");
            reads(f, launches);
            HIP_TRY(d, hipEventRecord(e1, s), "hipEventRecord");
            HIP_TRY(d, hipEventSynchronize(e1), "hipEventSynchronize");
            HIP_TRY(d, hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
            const float us = ms * 1e3f / launches;
            if (best == 0.0f || us < best) best = us;
        }
        *read_us = best;
        HIP_TRY(d, hipGetLastError(), "launch floor kernels");
        return RK_OK;
    };
    rc = run();
    (void)hipStreamSynchronize(s);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (sink) (void)hipFree(sink);
    if (buf) (void)hipFree(buf);
    return rc;
}
