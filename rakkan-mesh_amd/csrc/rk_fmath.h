// rk_fmath.h — device restatements of package num's float functions, for
// gfx950. Only correctly rounded f32/f64 additions and multiplications,
// integer operations and exact scalings are used (no v_rcp/v_rsq/v_exp, no
// fused multiply-add: every file including this is built with
// -ffp-contract=off), so each function gives the CPU's bits.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rk {

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// float32 roundings of the reference's untyped constants (exact rational,
// rounded once, as Go does).
constexpr uint32_t kCanonNaN = 0x7fc00000u;
constexpr uint32_t k1_127 = 0x3c010204u;  // internal/num/quant.go:42
constexpr uint32_t k24_17 = 0x3fb4b4b5u;  // internal/num/recip.go:54
constexpr uint32_t k8_17 = 0x3ef0f0f1u;   // internal/num/recip.go:54
constexpr uint32_t kLog2e = 0x3fb8aa3bu;  // internal/num/num.go:89
constexpr uint32_t kLn2Hi = 0x3f317200u;  // internal/num/num.go:86
constexpr uint32_t kLn2Lo = 0x35bfbe8eu;  // internal/num/num.go:87
constexpr uint32_t kExpHi = 0x42b170a4u;  // 88.72, internal/num/num.go:80
constexpr uint32_t kExpLo = 0xc2cff0a4u;  // -103.97, internal/num/num.go:82

// internal/num/num.go:26-31 Canonical.
__device__ __forceinline__ float canonical(float v) { return v != v ? u2f(kCanonNaN) : v; }

// Go's max for floats: NaN if either is NaN, +0 for (-0, +0).
__device__ __forceinline__ float gomax(float x, float y) {
    if (x != x || y != y) return u2f(kCanonNaN);
    if (x > y) return x;
    if (y > x) return y;
    return u2f(f2u(x) & f2u(y));
}

// internal/num/recip.go:16 Pow2, k in [-126, 127].
__device__ __forceinline__ float pow2(int k) { return u2f((uint32_t)(k + 127) << 23); }

// internal/num/recip.go:21-24 Scale2.
__device__ __forceinline__ float scale2(float v, int k) {
    int k1 = k / 2;
    float t = v * pow2(k1);
    return t * pow2(k - k1);
}

// internal/num/recip.go:27-35 split, positive finite x.
__device__ __forceinline__ float split(float x, int &e) {
    uint32_t b = f2u(x);
    int ee = 0;
    if ((b >> 23) == 0) {
        b = f2u(x * pow2(64));
        ee = -64;
    }
    e = ee + (int)(b >> 23) - 127;
    return u2f((b & 0x7fffffu) | (127u << 23));
}

// internal/num/recip.go:38-67 Recip32, without branches: the main path runs
// for every input and the special cases (NaN, ±0, ±Inf; a subnormal input's
// scaling into the normal range; Scale2 for a result outside it) are picked
// by selects, so the code is one straight run (a one-time prologue pays for
// every branch target it has to fetch). Pow2's argument is out of range only
// on the paths the selects discard.
__device__ __forceinline__ float recip32(float x) {
    const uint32_t bx = f2u(x);
    const uint32_t sign = bx & 0x80000000u;
    const uint32_t ab = bx & 0x7fffffffu;
    const bool sub = (ab >> 23) == 0;
    const uint32_t b = sub ? f2u(u2f(ab) * pow2(64)) : ab;
    const int e = (sub ? -64 : 0) + (int)(b >> 23) - 127;
    const float m = u2f((b & 0x7fffffu) | (127u << 23));
    float r = u2f(k24_17) - (u2f(k8_17) * m);
#pragma unroll
    for (int i = 0; i < 3; i++) {
        float mr = m * r;
        float t = r * (1.0f - mr);
        r = r + t;
    }
    const int k = -e, k1 = k / 2;
    const float rs = (r * pow2(k1)) * pow2(k - k1);  // Scale2(r, -e)
    const float rd = r * pow2(k);
    r = (e > 126 || e < -127) ? rs : rd;
    const uint32_t out = ab > 0x7f800000u ? kCanonNaN : ab == 0 ? (sign | 0x7f800000u) : ab == 0x7f800000u ? sign : (f2u(r) | sign);
    return u2f(out);
}

// internal/num/recip.go:70-93 Rsqrt32.
__device__ __forceinline__ float rsqrt32(float x) {
    if (x != x || x < 0.0f) return u2f(kCanonNaN);
    if (x == 0.0f) return __builtin_inff();
    if (x == __builtin_inff()) return 0.0f;
    int e;
    float m = split(x, e);
    if (e & 1) {
        m = m * 2.0f;
        e = e - 1;
    }
    float r = u2f(0x5f3759dfu - (f2u(m) >> 1));
    float h = 0.5f * m;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float t = (h * r) * r;
        r = r + r * (0.5f - t);
    }
    return r * pow2(-e / 2);
}

// internal/num/num.go:76-97 Exp32. math.Ldexp then the float32 conversion:
// the scaling is exact in f64 and the conversion rounds once (to a denormal
// if need be; f32 denormals are kept on gfx950).
__device__ __forceinline__ float exp32(float x) {
    if (x != x) return u2f(kCanonNaN);
    if (x > u2f(kExpHi)) return __builtin_inff();
    if (x < u2f(kExpLo)) return 0.0f;
    float n = __builtin_rintf(x * u2f(kLog2e));
    float r = x - (n * u2f(kLn2Hi));
    r = r - (n * u2f(kLn2Lo));
    float p = u2f(0x3ab60b61u);            // 1/720
    p = (p * r) + u2f(0x3c088889u);        // 1/120
    p = (p * r) + u2f(0x3d2aaaabu);        // 1/24
    p = (p * r) + u2f(0x3e2aaaabu);        // 1/6
    p = (p * r) + 0.5f;
    p = (p * r) + 1.0f;
    p = (p * r) + 1.0f;
    return (float)__builtin_ldexp((double)p, (int)n);
}

// Q8_0 code of v at inverse scale id: internal/num/quant.go:50,
// int8(max(-127, min(127, RoundToEven(float32(v*id))))); a NaN product
// (0·Inf, from a denormal scale) gives 0, as amd64's conversion does.
__device__ __forceinline__ int q8_code(float v, float id) {
    const float r = __builtin_rintf(v * id);
    const float c = __builtin_amdgcn_fmed3f(r, -127.0f, 127.0f);  // exact: the middle of r and the bounds
    return r != r ? 0 : (int)c;
}

// Go's max of the magnitudes |a|, |b|, |c| and m (m >= +0 or NaN): gfx950's
// IEEE maximum propagates NaN and orders -0 below +0, which is Go max on
// these operands except for which NaN it returns (the callers canonicalize).
__device__ __forceinline__ float abs_max3(float m, float a, float b) {
    return __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(fabsf(a), fabsf(b)));
}

}  // namespace rk
