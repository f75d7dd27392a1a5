// rk_num.hip — rk_num_eval: the device restatements of package num's float
// functions (rk_fmath.h) applied elementwise, so host callers get exactly
// what the kernels compute (and tests can compare them with the CPU's).
#include "rk_dev.h"
#include "rk_runtime.h"

namespace rk {

__global__ void num_eval_kernel(int fn, const float *in, float *out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = in[i];
    float y;
    switch (fn) {
        case RK_FN_RECIP32: y = recip32(x); break;
        case RK_FN_RSQRT32: y = rsqrt32(x); break;
        case RK_FN_EXP32: y = exp32(x); break;
        default: y = silu_mul(x, 1.0f); break;  // silu(x)·1 = silu(x) exactly
    }
    out[i] = y;
}

}  // namespace rk

using namespace rk;

extern "C" int rk_num_eval(rk_device *d, int32_t fn, const float *in, float *out, int64_t n) {
    if (!d || n < 0 || (n > 0 && (!in || !out)) || fn < RK_FN_RECIP32 || fn > RK_FN_SILU)
        return fail(d, RK_ERR_ARGS, "rk_num_eval: bad arguments");
    if (n == 0) return RK_OK;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    float *buf = nullptr;
    int rc = dev_alloc(d, (void **)&buf, (size_t)n * 8, "num_eval");
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(buf, in, (size_t)n * 4, hipMemcpyHostToDevice, d->stream);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(num_eval_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, d->stream, (int)fn, buf,
                           buf + n, n);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpyAsync(out, buf + n, (size_t)n * 4, hipMemcpyDeviceToHost, d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    (void)hipFree(buf);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return hip_fail(d, e, "rk_num_eval");
    }
    return RK_OK;
}
