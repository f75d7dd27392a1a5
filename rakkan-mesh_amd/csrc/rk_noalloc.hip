// rk_noalloc.hip — rk_matmul_t_device_noalloc: the batched products of
// rk_matmul_t_device for callers that cannot allocate device memory (code
// under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
//
// rk_matmul_t_device keeps the tokens' quantized inputs in a device scratch
// that it grows with hipMalloc when a call needs more. This variant keeps
// them in `scratch`, a file-scope device array of fixed size, and never
// allocates: tokens·cols is limited to kNoAllocCodes (2^24 codes: 512
// tokens of up to 32768 columns), checked before anything is enqueued.
//
// In host code `scratch` names a host-side stand-in, not device memory, so
// its device address is looked up once per device when the device is opened
// (noalloc_setup, with that device current) and kept in the rk_device; the
// kernels receive that address. Each GPU holds its own copy of the array
// (about 20 MiB) until the process ends.
//
// Every call on a device uses the same array, and each call's quantize
// kernel overwrites all of the codes, scales and code sums its products
// read, so no part of the array needs clearing. Calls that overlap on one
// device (enqueued on different streams without an order between them, or
// replays of graphs holding them on different streams) race on the array:
// the caller orders them, for example by using one stream.
#include "rk_mm.h"
#include "rk_runtime.h"

namespace rk {

constexpr int64_t kNoAllocCodes = (int64_t)1 << 24;
constexpr int64_t kNoAllocBlocks = kNoAllocCodes / 32;
// codes [kNoAllocCodes] int8, then scales [kNoAllocBlocks] f32, then code
// sums [kNoAllocBlocks] i32
constexpr int64_t kNoAllocBytes = kNoAllocCodes + 8 * kNoAllocBlocks;

static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

int noalloc_setup(rk_device *d) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return fail(d, RK_ERR_HIP, "static scratch: hipGetSymbolAddress: %s", hipGetErrorString(e));
    }
    d->noalloc = p;
    return RK_OK;
}

}  // namespace rk

using namespace rk;

extern "C" int rk_matmul_t_device_noalloc(rk_device *d, int32_t n, rk_matrix *const *ms, float *const *d_outs,
                                          const float *d_x, int64_t cols, int32_t tokens, void *stream) {
    int64_t total;
    int rc = check_matmul(d, n, ms, cols, tokens, &total);
    if (rc) return rc;
    if (n == 0 || tokens == 0) return RK_OK;
    if (!d_x || !d_outs) return fail(d, RK_ERR_ARGS, "rk_matmul_t_device_noalloc: null buffer");
    for (int i = 0; i < n; i++)
        if (!d_outs[i]) return fail(d, RK_ERR_ARGS, "rk_matmul_t_device_noalloc: null output %d", i);
    if ((int64_t)tokens * cols > kNoAllocCodes)
        return fail(d, RK_ERR_ARGS,
                    "rk_matmul_t_device_noalloc: %d tokens of %lld columns exceed the static scratch of %lld codes",
                    tokens, (long long)cols, (long long)kNoAllocCodes);
    if (!d->noalloc) return fail(d, RK_ERR_HIP, "rk_matmul_t_device_noalloc: the static scratch has no address");
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    hipStream_t s = stream ? (hipStream_t)stream : d->stream;
    if (d->capturing && s != d->stream)
        return fail(d, RK_ERR_ARGS, "while recording a graph, work goes on the device's stream");
    uint8_t *base = static_cast<uint8_t *>(d->noalloc);
    const QScratch q{reinterpret_cast<int8_t *>(base), reinterpret_cast<float *>(base + kNoAllocCodes),
                     reinterpret_cast<int32_t *>(base + kNoAllocCodes + 4 * kNoAllocBlocks)};
    return enqueue_matmuls(d, n, ms, d_outs, d_x, cols, tokens, q, s);
}
