// rk_matvec.hip — the activation quantizer of the products that take a
// separately quantized input (rk_fused.hip kProGlobal): x -> Q8_0 codes,
// block scales and block code sums (internal/num/quant.go:34-53).
#include "rk_dev.h"
#include "rk_kernels.h"

namespace rk {

// ---------------------------------------------------------------------------
// Activation quantize: internal/num/quant.go:34-53, eight lanes per block.
__global__ __launch_bounds__(256) void quantize_acts_kernel(const float *x, int64_t nb, int8_t *qx, float *xs,
                                                            int32_t *xsum) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t b = t >> 3;
    const bool ok = b < nb;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (ok) {  // x may be only 4-byte aligned (an arena word offset)
        const float *p = x + t * 4;
        v = make_float4(p[0], p[1], p[2], p[3]);
    }
    float d;
    int s;
    const uint32_t packed = quantize_group(v.x, v.y, v.z, v.w, d, s);
    if (ok) {
        reinterpret_cast<uint32_t *>(qx)[t] = packed;
        if ((threadIdx.x & 7) == 0) {
            xs[b] = d;
            xsum[b] = s;
        }
    }
}

void launch_quantize_acts(const float *x, int64_t n, int8_t *qx, float *xs, int32_t *xsum, hipStream_t s) {
    const int64_t nb = n / 32;
    if (nb <= 0) return;
    const int64_t threads = nb * 8;
    RK_LAUNCH(quantize_acts_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, x, nb, qx, xs,
                       xsum);
}

}  // namespace rk
