/*
 * rk_oracle_mx.c — CPU restatement of DeepSeek-V4.1's block-scaled
 * ("microscaling") arithmetic, internal/num/mx.go. TEST INFRASTRUCTURE ONLY
 * (see rk_oracle.h).
 *
 * E4M3: sign, 4 exponent bits (bias 7), 3 mantissa bits, no infinities,
 * 0x7f / 0xff NaN. E2M1: sign, 2 exponent bits, 1 mantissa bit, magnitudes
 * 0, .5, 1, 1.5, 2, 3, 4, 6, two to a byte (even element low). E8M0: 2^(c-127),
 * 0 is 2^-127, 255 NaN.
 *
 * A block's 32 products are exact in float64 (E4M3 x E4M3) or int32 (E2M1 x
 * E4M3, twice the weight times 512 times the input), so any summation order
 * gives the same block sum; the blocks' terms are then added in order in
 * float32 (mx.go:371-388 combineBlocks).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "rk_oracle.h"

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static const float FP4_GRID[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

/* mx.go:48-66 init: the value of an E4M3 code (NaN codes: NaN). */
double rko_e4m3_value(uint8_t c) {
    int sign = c >> 7, e = (c >> 3) & 15, m = c & 7;
    double v;
    if (e == 15 && m == 7)
        v = NAN;
    else if (e == 0)
        v = ldexp((double)m, -9);
    else
        v = ldexp((double)(8 + m), e - 10);
    return sign ? -v : v;
}

/* The 256 codes' values, filled once (mx.go:34-36 e4m3F64). */
static double E4M3[256];
static int e4m3_ready;
static const double *e4m3_table(void) {
    if (!e4m3_ready) {
        for (int c = 0; c < 256; c++) E4M3[c] = rko_e4m3_value((uint8_t)c);
        e4m3_ready = 1;
    }
    return E4M3;
}

/* mx.go:90-111 EncodeE4M3: nearest E4M3 value, ties to even; beyond 448
 * saturates to 0x7e; NaN is 0x7f. */
uint8_t rko_encode_e4m3(float v) {
    if (v != v) return 0x7f;
    uint8_t sign = signbit(v) ? 0x80 : 0;
    double a = fabs((double)v);
    if (a < 1.0 / 64) return sign | (uint8_t)nearbyint(a * 512); /* 8 is the smallest normal's code */
    int x;
    (void)frexp(a, &x); /* a = f 2^x, f in [0.5, 1) */
    int e = x - 1;
    double n = nearbyint(ldexp(a, 3 - e));
    if (n == 16) {
        e++;
        n = 8;
    }
    int code = (e + 7) << 3 | ((int)n - 8);
    return sign | (uint8_t)(code < 0x7e ? code : 0x7e);
}

/* mx.go:113-124 DecodeE8M0 */
float rko_decode_e8m0(uint8_t c) {
    if (c == 255) return u2f(0x7fc00000u);
    if (c == 0) return u2f(1u << 22);
    return u2f((uint32_t)c << 23);
}

/* mx.go:126 DecodeE2M1 */
float rko_decode_e2m1(uint8_t c) {
    float v = FP4_GRID[c & 7];
    return (c & 8) ? -v : v;
}

/* EncodeE4M3 over an array. */
void rko_encode_e4m3_n(const float *v, int64_t n, uint8_t *out) {
    for (int64_t i = 0; i < n; i++) out[i] = rko_encode_e4m3(v[i]);
}

/* mx.go:128-145 EncodeE2M1: nearest, ties to the even code, sign kept. */
uint8_t rko_encode_e2m1(float v) {
    float a = fabsf(v);
    uint8_t code = 0;
    for (int i = 0; i < 7; i++) {
        float mid = (FP4_GRID[i] + FP4_GRID[i + 1]) / 2;
        if (a > mid || (a == mid && (i + 1) % 2 == 0)) code = (uint8_t)(i + 1);
    }
    if (signbit(v)) code |= 8;
    return code;
}

/* mx.go:147-156 pow2Ceil: the exponent field plus one if any mantissa bit
 * is set, as bits (uint32 arithmetic: a NaN gives 2^31, -0). */
float rko_pow2ceil(float t) {
    uint32_t b = f2u(t);
    int32_t e = (int32_t)((b >> 23) & 0xff) - 127;
    if (b & 0x7fffff) e++;
    return u2f((uint32_t)(e + 127) << 23);
}

/* Go's builtin min / max on float32: NaN if either is NaN. */
static inline float go_max(float x, float y) {
    if (x != x || y != y) return u2f(0x7fc00000u);
    if (x > y) return x;
    if (y > x) return y;
    return u2f(f2u(x) & f2u(y));
}
static inline float go_min(float x, float y) {
    if (x != x || y != y) return u2f(0x7fc00000u);
    if (x < y) return x;
    if (y < x) return y;
    return u2f(f2u(x) | f2u(y));
}

/* mx.go:158-164 absMax */
static float abs_max(const float *x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; i++) m = go_max(m, fabsf(x[i]));
    return m;
}

/* mx.go:185-203 QuantizeActFP8: per block of 32, s = pow2Ceil(max(amax,
 * float32(1e-4)) * float32(1/448)), codes = EncodeE4M3(clamp(v / s, ±448)).
 * codes[i] is the E4M3 code of element i (the value ActFP8.Vals holds). */
void rko_act_fp8(const float *x, int64_t n, uint8_t *codes, float *scales) {
    const float inv448 = (float)(1.0 / 448), floor_ = (float)1e-4;
    for (int64_t b = 0; b < n / 32; b++) {
        const float *blk = x + b * 32;
        volatile float t = go_max(abs_max(blk, 32), floor_) * inv448;
        float s = rko_pow2ceil(t);
        scales[b] = s;
        for (int j = 0; j < 32; j++) {
            volatile float q = blk[j] / s;
            codes[b * 32 + j] = rko_encode_e4m3(go_min(go_max(q, -448.0f), 448.0f));
        }
    }
}

/* mx.go:205-214 ActQuantInPlace: each value its E4M3 rounding times the
 * block scale, in bfloat16. */
void rko_act_quant_inplace(float *x, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        uint8_t c[32];
        float s;
        rko_act_fp8(x + b * 32, 32, c, &s);
        for (int j = 0; j < 32; j++) {
            volatile float v = (float)rko_e4m3_value(c[j]) * s;
            x[b * 32 + j] = rko_bf16(rko_to_bf16(v));
        }
    }
}

/* The input's E4M3 value times 512 as Go's int32(q * 512) gives it on
 * x86-64 (mx.go:200): an integer below 2^18 in magnitude, or, for a NaN
 * code, the conversion's integer indefinite 0x80000000. */
static int32_t x_int(uint8_t c) {
    double q = rko_e4m3_value(c);
    if (q != q) return INT32_MIN;
    return (int32_t)(q * 512);
}

/* mx.go:371-388 combineBlocks: each block's exact sum times unit rounded to
 * float32, times the input's scale, times the weight's, added in order;
 * NaN canonical; then bfloat16 if asked. */
static float combine_blocks(const double *sums, const float *xs, const uint8_t *ws, int64_t nb, double unit,
                            int bf16) {
    float acc = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        volatile float t = (float)(sums[b] * unit);
        t = t * xs[b];
        t = t * rko_decode_e8m0(ws[b]);
        acc = acc + t;
    }
    acc = rko_canonical(acc);
    if (bf16) acc = rko_bf16(rko_to_bf16(acc));
    return acc;
}

/* mx.go:282-296 MatVecFP8 (bf16 = 1) / MatVecFP8Unrounded (bf16 = 0): E4M3
 * weights [rows][cols], E8M0 scales [ceil(rows/32)][cols/32]; the input as
 * rko_act_fp8 leaves it (codes and block scales). Block sums in float64
 * (mx.go:399-410 blockDotFP8; exact, so the order is free). */
void rko_matvec_fp8(float *out, const uint8_t *w, const uint8_t *ws, const uint8_t *xc, const float *xs, int64_t rows,
                    int64_t cols, int bf16) {
    int64_t nb = cols / 32;
    const double *tab = e4m3_table();
    double *xv = malloc(sizeof(double) * (size_t)(cols + 1)), *sums = malloc(sizeof(double) * (size_t)(nb + 1));
    for (int64_t j = 0; j < cols; j++) xv[j] = tab[xc[j]];
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t *row = w + r * cols;
        for (int64_t b = 0; b < nb; b++) {
            double s = 0;
            for (int j = 0; j < 32; j++) s += tab[row[b * 32 + j]] * xv[b * 32 + j];
            sums[b] = s;
        }
        out[r] = combine_blocks(sums, xs, ws + (r / 32) * nb, nb, 1.0, bf16);
    }
    free(xv);
    free(sums);
}

/* mx.go:315-334, 390-397 MatVecFP4: E2M1 codes packed [rows][cols/2], E8M0
 * scales [rows][cols/32]. A block's sum is the int32 dot product of twice
 * the weights and the input times 512 (wrapping, as Go's int32 does), then
 * times 1/1024. */
void rko_matvec_fp4(float *out, const uint8_t *w, const uint8_t *ws, const uint8_t *xc, const float *xs, int64_t rows,
                    int64_t cols, int bf16) {
    int64_t nb = cols / 32;
    double *sums = malloc(sizeof(double) * (size_t)(nb + 1));
    int32_t *xi = malloc(sizeof(int32_t) * (size_t)(cols + 1));
    for (int64_t j = 0; j < cols; j++) xi[j] = x_int(xc[j]);
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t *row = w + r * (cols / 2);
        for (int64_t b = 0; b < nb; b++) {
            uint32_t s = 0;
            for (int j = 0; j < 32; j++) {
                uint8_t c = (row[b * 16 + j / 2] >> (4 * (j & 1))) & 15;
                int32_t w2 = (int32_t)(2 * rko_decode_e2m1(c));
                s += (uint32_t)w2 * (uint32_t)xi[b * 32 + j];
            }
            sums[b] = (double)(int32_t)s;
        }
        out[r] = combine_blocks(sums, xs, ws + r * nb, nb, 1.0 / 1024, bf16);
    }
    free(sums);
    free(xi);
}

/* mx.go:234-266 QuantizeFP4: blocks of 32 with E8M0 scales (e4m3 = 0) or of
 * 16 with E4M3 scales (e4m3 = 1); packed len(x)/2 bytes, one scale byte a
 * block. */
void rko_quantize_fp4(const float *x, int64_t n, int e4m3, uint8_t *packed, uint8_t *scales) {
    const int blk = e4m3 ? 16 : 32;
    const float inv6 = (float)(1.0 / 6);
    for (int64_t b = 0; b < n / blk; b++) {
        const float *vals = x + b * blk;
        float amax = abs_max(vals, blk);
        volatile float s;
        if (e4m3) {
            amax = go_max(amax, 6 * (1.0f / 512));
            volatile float t = amax / 6;
            scales[b] = rko_encode_e4m3(t);
            s = (float)rko_e4m3_value(scales[b]);
        } else {
            amax = go_max(amax, (float)ldexp(6, -126));
            volatile float t = amax * inv6;
            s = rko_pow2ceil(t);
            scales[b] = (uint8_t)(f2u(s) >> 23);
        }
        for (int j = 0; j < blk; j++) {
            volatile float q = vals[j] / s;
            uint8_t c = rko_encode_e2m1(go_min(go_max(q, -6.0f), 6.0f));
            int64_t i = b * blk + j;
            if (i % 2 == 0)
                packed[i / 2] = c;
            else
                packed[i / 2] |= (uint8_t)(c << 4);
        }
    }
}

/* mx.go:268-280 DequantFP4 */
void rko_dequant_fp4(float *x, int64_t n, int e4m3, const uint8_t *packed, const uint8_t *scales) {
    const int blk = e4m3 ? 16 : 32;
    for (int64_t i = 0; i < n; i++) {
        float s = e4m3 ? (float)rko_e4m3_value(scales[i / blk]) : rko_decode_e8m0(scales[i / blk]);
        volatile float v = rko_decode_e2m1((packed[i / 2] >> (4 * (i % 2))) & 15) * s;
        x[i] = rko_bf16(rko_to_bf16(v));
    }
}
