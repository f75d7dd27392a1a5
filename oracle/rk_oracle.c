/*
 * rk_oracle.c — CPU restatement of rakkan-mesh's deterministic arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP backend (see rk_oracle.h).
 *
 * Reference paths are relative to the rakkan-mesh repository. Go rules that
 * this C code reproduces:
 *   - an untyped constant meeting a float32 operand is rounded to float32
 *     once; the constants below are written as their float32 bit patterns
 *     (the test suite re-derives each from the exact rational);
 *   - float32(x*y) rounds the product, so nothing is fused (built with
 *     -ffp-contract=off, and no FMA target feature is enabled);
 *   - Go's max for floats: NaN if either argument is, and +0 over -0.
 */
#include "rk_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }

#define CANON_NAN 0x7fc00000u
/* float32 roundings of the Go constants (exact rational, rounded once). */
#define K_1_127   0x3c010204u /* 1.0/127            quant.go:42        */
#define K_24_17   0x3fb4b4b5u /* 24.0/17            recip.go:54        */
#define K_8_17    0x3ef0f0f1u /* 8.0/17             recip.go:54        */
#define K_LOG2E   0x3fb8aa3bu /* 1.4426950408889634 num.go:89          */
#define K_LN2HI   0x3f317200u /* 0.693145751953125  num.go:86          */
#define K_LN2LO   0x35bfbe8eu /* 1.428606765330187e-06 num.go:87       */
#define K_1_720   0x3ab60b61u /* 1.0/720            num.go:92          */
#define K_1_120   0x3c088889u
#define K_1_24    0x3d2aaaabu
#define K_1_6     0x3e2aaaabu
#define K_EXP_HI  0x42b170a4u /* 88.72   num.go:80 */
#define K_EXP_LO  0xc2cff0a4u /* -103.97 num.go:82 */

/* ------------------------------------------------------------------ */
/* internal/num/num.go:26-31 Canonical                                 */
float rko_canonical(float v) { return v != v ? u2f(CANON_NAN) : v; }

/* Go's builtin max for float32 (Go spec, "Min and max"). */
float rko_gomax(float x, float y) {
    if (x != x || y != y) return u2f(CANON_NAN);
    if (x > y) return x;
    if (y > x) return y;
    return u2f(f2u(x) & f2u(y)); /* equal: +0 wins over -0 */
}

/* internal/num/recip.go:16 Pow2 */
float rko_pow2(int k) { return u2f((uint32_t)(k + 127) << 23); }

/* internal/num/recip.go:21-24 Scale2 */
float rko_scale2(float v, int k) {
    int k1 = k / 2; /* Go's / truncates toward zero, as C's */
    float t = v * rko_pow2(k1);
    return t * rko_pow2(k - k1);
}

/* internal/num/recip.go:27-35 split */
static float split32(float x, int *e) {
    uint32_t b = f2u(x);
    int ee = 0;
    if ((b >> 23) == 0) {
        b = f2u(x * rko_pow2(64));
        ee = -64;
    }
    ee += (int)(b >> 23) - 127;
    *e = ee;
    return u2f((b & 0x7fffffu) | (127u << 23));
}

/* internal/num/recip.go:38-67 Recip32 */
float rko_recip32(float x) {
    if (x != x) return u2f(CANON_NAN);
    if (x == 0) return (f2u(x) >> 31) ? -INFINITY : INFINITY;
    if (isinf(x)) return (f2u(x) >> 31) ? -0.0f : 0.0f;
    int neg = x < 0;
    if (neg) x = -x;
    int e;
    float m = split32(x, &e);
    float r = u2f(K_24_17) - (u2f(K_8_17) * m);
    for (int i = 0; i < 3; i++) {
        float mr = m * r;
        float t = r * (1.0f - mr);
        r = r + t;
    }
    if (e > 126 || e < -127)
        r = rko_scale2(r, -e);
    else
        r = r * rko_pow2(-e);
    if (neg) r = -r;
    return r;
}

/* internal/num/recip.go:70-93 Rsqrt32 */
float rko_rsqrt32(float x) {
    if (x != x || x < 0) return u2f(CANON_NAN);
    if (x == 0) return INFINITY;
    if (isinf(x)) return 0.0f;
    int e;
    float m = split32(x, &e);
    if (e & 1) {
        m = m * 2.0f;
        e = e - 1;
    }
    float r = u2f(0x5f3759dfu - (f2u(m) >> 1));
    float h = 0.5f * m;
    for (int i = 0; i < 4; i++) {
        float t = (h * r) * r;
        r = r + r * (0.5f - t);
    }
    return r * rko_pow2(-e / 2);
}

/* internal/num/num.go:76-97 Exp32 */
float rko_exp32(float x) {
    if (x != x) return u2f(CANON_NAN);
    if (x > u2f(K_EXP_HI)) return INFINITY;
    if (x < u2f(K_EXP_LO)) return 0.0f;
    float n = (float)rint((double)(x * u2f(K_LOG2E)));
    float r = x - (n * u2f(K_LN2HI));
    r = r - (n * u2f(K_LN2LO));
    static const uint32_t cs[6] = {K_1_120, K_1_24, K_1_6, 0x3f000000u, 0x3f800000u, 0x3f800000u};
    float p = u2f(K_1_720);
    for (int i = 0; i < 6; i++) p = (p * r) + u2f(cs[i]);
    return (float)ldexp((double)p, (int)n);
}

static double factorial(int k) {
    double f = 1.0;
    for (int i = 2; i <= k; i++) f *= (double)i;
    return f;
}

/* internal/num/num.go:101-123 Exp (float64) */
double rko_exp(double x) {
    if (x != x) return x;
    if (x > 709.78) return INFINITY;
    if (x < -745.13) return 0.0;
    const double ln2Hi = 6.93147180369123816490e-01, ln2Lo = 1.90821492927058770002e-10;
    double n = rint(x * 1.4426950408889634);
    double r = x - (n * ln2Hi);
    r = r - (n * ln2Lo);
    double p = 1.0 / 6227020800.0;
    for (int k = 12; k >= 0; k--) p = (p * r) + 1.0 / factorial(k);
    return ldexp(p, (int)n);
}

/* internal/num/num.go:128-163 Log (fdlibm, as Go's math.Log) */
double rko_log(double x) {
    const double ln2Hi = 6.93147180369123816490e-01, ln2Lo = 1.90821492927058770002e-10;
    const double l1 = 6.666666666666735130e-01, l2 = 3.999999999940941908e-01, l3 = 2.857142874366239149e-01,
                 l4 = 2.222219843214978396e-01, l5 = 1.818357216161805012e-01, l6 = 1.531383769920937332e-01,
                 l7 = 1.479819860511658591e-01;
    if (x != x || (isinf(x) && x > 0)) return x;
    if (x < 0) return NAN;
    if (x == 0) return -INFINITY;
    int ki;
    double f1 = frexp(x, &ki);
    if (f1 < 0.70710678118654752440 /* math.Sqrt2/2 */) {
        f1 *= 2;
        ki--;
    }
    double f = f1 - 1;
    double k = (double)ki;
    double s = f / (2 + f);
    double s2 = s * s;
    double s4 = s2 * s2;
    double t1 = s2 * (l1 + (s4 * (l3 + (s4 * (l5 + (s4 * l7))))));
    double t2 = s4 * (l2 + (s4 * (l4 + (s4 * l6))));
    double r = t1 + t2;
    double hfsq = (0.5 * f) * f;
    return (k * ln2Hi) - ((hfsq - ((s * (hfsq + r)) + (k * ln2Lo))) - f);
}

/* internal/num/num.go:169-207 Log32 */
float rko_log32(float x) {
    const float ln2Hi = 6.9313812256e-01f, ln2Lo = 9.0580006145e-06f, lg1 = 6.6666662693e-01f,
                lg2 = 4.0000972152e-01f, lg3 = 2.8498786688e-01f, lg4 = 2.4279078841e-01f;
    if (x != x || (isinf(x) && x > 0)) return x;
    if (x < 0) return u2f(CANON_NAN);
    if (x == 0) return -INFINITY;
    uint32_t b = f2u(x);
    int32_t ki = (int32_t)(b >> 23) - 127;
    if ((b >> 23) == 0) {
        b = f2u(x * 16777216.0f);
        ki = (int32_t)(b >> 23) - 127 - 24;
    }
    float f1 = u2f((b & 0x7fffffu) | (127u << 23));
    if (f1 > 1.41421356237309504880f) {
        f1 = f1 * 0.5f;
        ki++;
    }
    float f = f1 - 1;
    float k = (float)ki;
    float s = f / (2 + f);
    float z = s * s;
    float w = z * z;
    float t1 = w * (lg2 + (w * lg4));
    float t2 = z * (lg1 + (w * lg3));
    float r = t2 + t1;
    float hfsq = (0.5f * f) * f;
    return (k * ln2Hi) - ((hfsq - ((s * (hfsq + r)) + (k * ln2Lo))) - f);
}

/* internal/num/num.go:224-231 Log1p (float64) */
double rko_log1p(double x) {
    double u = 1 + x;
    if (u == 1) return x;
    return (rko_log(u) * x) / (u - 1);
}

/* internal/num/num.go:244-297 Sincos with the Cephes polynomials */
static const double sin_coef[6] = {1.58962301576546568060e-10, -2.50507477628578072866e-8, 2.75573136213857245213e-6,
                                   -1.98412698295895385996e-4, 8.33333333332211858878e-3, -1.66666666666666307295e-1};
static const double cos_coef[6] = {-1.13585365213876817300e-11, 2.08757008419747316778e-9, -2.75573141792967388112e-7,
                                   2.48015872888517045348e-5, -1.38888888888730564116e-3, 4.16666666666665929218e-2};
static double sin_poly(double r) {
    double z = r * r;
    double p = sin_coef[0];
    for (int i = 1; i < 6; i++) p = (p * z) + sin_coef[i];
    return r + ((r * z) * p);
}
static double cos_poly(double r) {
    double z = r * r;
    double p = cos_coef[0];
    for (int i = 1; i < 6; i++) p = (p * z) + cos_coef[i];
    return 1 - (0.5 * z) + ((z * z) * p);
}
void rko_sincos(double x, double *sn, double *cs) {
    const double pio2a = 1.57079632673412561417e+00, pio2b = 6.07710050630396597660e-11,
                 pio2c = 2.02226624879595063154e-21;
    const double two_over_pi = 0.63661977236758134308; /* 2/math.Pi rounded to float64 */
    double k = rint(x * two_over_pi);
    double r = x - (k * pio2a);
    r = r - (k * pio2b);
    r = r - (k * pio2c);
    double s = sin_poly(r), c = cos_poly(r);
    switch (((int64_t)k) & 3) {
    case 0: *sn = s; *cs = c; break;
    case 1: *sn = c; *cs = -s; break;
    case 2: *sn = -s; *cs = -c; break;
    default: *sn = -c; *cs = s; break;
    }
}

/* internal/num/matvec.go:20-29 BF16 / ToBF16 */
float rko_bf16(uint16_t v) { return u2f((uint32_t)v << 16); }
uint16_t rko_to_bf16(float f) {
    uint32_t b = f2u(f);
    if (f != f) return (uint16_t)(b >> 16) | 0x40;
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1)) >> 16);
}

/* ------------------------------------------------------------------ */
/* internal/num/num.go:34-41 Dot: one chain in order */
float rko_dot(const float *a, const float *b, int64_t n) {
    float acc = 0.0f;
    for (int64_t i = 0; i < n; i++) acc += a[i] * b[i];
    return acc;
}

/* internal/num/matvec.go:60-66 combine */
static float combine32(const float s[32]) {
    float e[8];
    for (int j = 0; j < 8; j++) e[j] = (s[j] + s[j + 8]) + (s[j + 16] + s[j + 24]);
    return ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
}

/* internal/num/matvec.go:32-43 Dot32: element i into sum i mod 32 */
float rko_dot32(const float *a, const float *b, int64_t n) {
    float s[32];
    for (int j = 0; j < 32; j++) s[j] = 0.0f;
    for (int64_t i = 0; i < n; i++) s[i & 31] += a[i] * b[i];
    return combine32(s);
}

/* internal/num/matvec.go:47-58 DotBF16 */
float rko_dot_bf16(const uint16_t *w, const float *x, int64_t n) {
    float s[32];
    for (int j = 0; j < 32; j++) s[j] = 0.0f;
    for (int64_t i = 0; i < n; i++) s[i & 31] += rko_bf16(w[i]) * x[i];
    return combine32(s);
}

/* internal/num/matvec.go:106-123 MatVec32 / MatVecBF16 (split-independent) */
void rko_matvec32(float *out, const float *w, const float *x, int64_t rows, int64_t cols) {
    for (int64_t i = 0; i < rows; i++) out[i] = rko_dot32(w + i * cols, x, cols);
}
void rko_matvec_bf16(float *out, const uint16_t *w, const float *x, int64_t rows, int64_t cols) {
    for (int64_t i = 0; i < rows; i++) out[i] = rko_dot_bf16(w + i * cols, x, cols);
}

/* ------------------------------------------------------------------ */
/* internal/num/quant.go:34-53 quantize8 (QuantizeQ8, QuantizeActs) */
void rko_quantize8(const float *w, int64_t n, int8_t *q, float *scales) {
    int64_t nb = n / 32;
    for (int64_t b = 0; b < nb; b++) {
        const float *blk = w + b * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = rko_gomax(amax, fabsf(blk[j]));
        float d = amax * u2f(K_1_127);
        scales[b] = d;
        if (d == 0 || d != d) {
            memset(q + b * 32, 0, 32);
            continue;
        }
        float id = rko_recip32(d);
        for (int j = 0; j < 32; j++) {
            float t = blk[j] * id;
            double r = rint((double)t);
            /* Go: int8(max(-127, min(127, r))); a NaN product (0·Inf) gives
             * NaN, whose int8 conversion on amd64 is 0. */
            int8_t v;
            if (r != r)
                v = 0;
            else
                v = (int8_t)(r > 127 ? 127 : (r < -127 ? -127 : r));
            q[b * 32 + j] = v;
        }
    }
}

/* internal/num/quant.go:119-127 quant4 */
static void quant4(const float *blk, float d, int8_t vals[32]) {
    float id = 0.0f;
    if (d != 0) id = 1.0f / d;
    for (int j = 0; j < 32; j++) {
        double r = rint((double)(blk[j] * id));
        vals[j] = (int8_t)(r != r ? 0 : (r > 7 ? 7 : (r < -8 ? -8 : r)));
    }
}

/* internal/num/quant.go:62-116 QuantizeQ4 / quantize4 */
void rko_quantize4(const float *w, int64_t n, uint8_t *q, float *scales) {
    static const float divs[6] = {-8.0f, -7.5f, -7.0f, 7.0f, 7.5f, 6.5f};
    int64_t nb = n / 32;
    int8_t vals[32], best[32];
    for (int64_t b = 0; b < nb; b++) {
        const float *blk = w + b * 32;
        float amax = 0.0f, peak = 0.0f;
        for (int j = 0; j < 32; j++) {
            float a = fabsf(blk[j]);
            if (a > amax) {
                amax = a;
                peak = blk[j];
            }
        }
        double bestErr = INFINITY;
        float bestD = 0.0f;
        memset(best, 0, sizeof best);
        if (amax > 0 && amax == amax) {
            for (int di = 0; di < 6; di++) {
                float d = peak / divs[di];
                for (int it = 0; it < 3; it++) {
                    quant4(blk, d, vals);
                    double wq = 0, qq = 0;
                    for (int j = 0; j < 32; j++) {
                        wq += (double)blk[j] * (double)vals[j];
                        qq += (double)vals[j] * (double)vals[j];
                    }
                    if (qq == 0) break;
                    d = (float)(wq / qq);
                }
                quant4(blk, d, vals);
                double e = 0;
                for (int j = 0; j < 32; j++) {
                    double diff = (double)blk[j] - (double)((float)vals[j] * d);
                    e += diff * diff;
                }
                if (e < bestErr) {
                    bestErr = e;
                    bestD = d;
                    memcpy(best, vals, 32);
                }
            }
        }
        scales[b] = bestD;
        for (int j = 0; j < 16; j++) q[b * 16 + j] = (uint8_t)((uint8_t)(best[j] + 8) | (uint8_t)((best[j + 16] + 8) << 4));
    }
}

/* internal/num/quant.go:130-146 DequantQ8 / DequantQ4 */
void rko_dequant8(float *dst, const int8_t *q, const float *scales, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = (float)q[i] * scales[i / 32];
}
void rko_dequant4(float *dst, const uint8_t *q, const float *scales, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        float d = scales[b];
        for (int j = 0; j < 16; j++) {
            uint8_t v = q[b * 16 + j];
            dst[b * 32 + j] = (float)((int)(v & 15) - 8) * d;
            dst[b * 32 + j + 16] = (float)((int)(v >> 4) - 8) * d;
        }
    }
}

/* internal/num/quant.go:198-218 blockSumsQ8Generic / blockSumsQ4Generic */
void rko_blocksums_q8(const int8_t *w, const int8_t *x, int64_t nb, int32_t *sums) {
    for (int64_t b = 0; b < nb; b++) {
        int32_t s = 0;
        for (int j = 0; j < 32; j++) s += (int32_t)w[b * 32 + j] * (int32_t)x[b * 32 + j];
        sums[b] = s;
    }
}
void rko_blocksums_q4(const uint8_t *w, const int8_t *x, int64_t nb, int32_t *sums) {
    for (int64_t b = 0; b < nb; b++) {
        int32_t s = 0;
        for (int j = 0; j < 16; j++) {
            uint8_t v = w[b * 16 + j];
            s += ((int32_t)(v & 15) - 8) * (int32_t)x[b * 32 + j] + ((int32_t)(v >> 4) - 8) * (int32_t)x[b * 32 + j + 16];
        }
        sums[b] = s;
    }
}

/* internal/num/quant.go:158-164 qrow: block b into lane b mod 8, fixed tree */
float rko_qrow(const int32_t *sums, const float *ws, const float *xs, int64_t nb) {
    float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t b = 0; b < nb; b++) {
        float d = ws[b] * xs[b];
        float t = (float)sums[b] * d;
        s[b & 7] += t;
    }
    return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

/* internal/num/quant.go:167-196 MatVecQ8 / MatVecQ4 */
void rko_matvec_q8(float *out, const int8_t *w, const float *ws, const float *x, int64_t rows, int64_t cols) {
    int64_t nb = cols / 32;
    int8_t *qx = malloc((size_t)cols);
    float *xs = malloc((size_t)nb * 4);
    int32_t *sums = malloc((size_t)nb * 4);
    rko_quantize8(x, cols, qx, xs);
    for (int64_t i = 0; i < rows; i++) {
        rko_blocksums_q8(w + i * cols, qx, nb, sums);
        out[i] = rko_qrow(sums, ws + i * nb, xs, nb);
    }
    free(qx); free(xs); free(sums);
}
void rko_matvec_q4(float *out, const uint8_t *w, const float *ws, const float *x, int64_t rows, int64_t cols) {
    int64_t nb = cols / 32;
    int8_t *qx = malloc((size_t)cols);
    float *xs = malloc((size_t)nb * 4);
    int32_t *sums = malloc((size_t)nb * 4);
    rko_quantize8(x, cols, qx, xs);
    for (int64_t i = 0; i < rows; i++) {
        rko_blocksums_q4(w + i * cols / 2, qx, nb, sums);
        out[i] = rko_qrow(sums, ws + i * nb, xs, nb);
    }
    free(qx); free(xs); free(sums);
}
void rko_matmul_q8(float *out, const int8_t *w, const float *ws, const float *x, int64_t tokens, int64_t rows, int64_t cols) {
    for (int64_t t = 0; t < tokens; t++) rko_matvec_q8(out + t * rows, w, ws, x + t * cols, rows, cols);
}
void rko_matmul_q4(float *out, const uint8_t *w, const float *ws, const float *x, int64_t tokens, int64_t rows, int64_t cols) {
    for (int64_t t = 0; t < tokens; t++) rko_matvec_q4(out + t * rows, w, ws, x + t * cols, rows, cols);
}

/* ------------------------------------------------------------------ */
/* CPU baseline: internal/num/dot_amd64.s:98-213 (4 blocks per step with
 * sign/maddubs/madd), rows split over threads as internal/num/matvec.go:90-104. */
#include <immintrin.h>

int rko_have_avx2(void) { return __builtin_cpu_supports("avx2"); }

__attribute__((target("avx2"))) static inline int32_t hsum8(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_hadd_epi32(s, s);
    s = _mm_hadd_epi32(s, s);
    return _mm_cvtsi128_si32(s);
}

__attribute__((target("avx2"))) static inline __m256i dot32_i8(__m256i w, __m256i x) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256i aw = _mm256_sign_epi8(w, w);
    __m256i sx = _mm256_sign_epi8(x, w);
    return _mm256_madd_epi16(_mm256_maddubs_epi16(aw, sx), ones);
}

__attribute__((target("avx2"))) static void blocksums_q8_avx2(const int8_t *w, const int8_t *x, int64_t nb, int32_t *sums) {
    int64_t b = 0;
    for (; b + 4 <= nb; b += 4)
        for (int k = 0; k < 4; k++) {
            __m256i wv = _mm256_loadu_si256((const __m256i *)(w + (b + k) * 32));
            __m256i xv = _mm256_loadu_si256((const __m256i *)(x + (b + k) * 32));
            sums[b + k] = hsum8(dot32_i8(wv, xv));
        }
    if (b < nb) rko_blocksums_q8(w + b * 32, x + b * 32, nb - b, sums + b);
}

__attribute__((target("avx2"))) static void blocksums_q4_avx2(const uint8_t *w, const int8_t *x, int64_t nb, int32_t *sums) {
    const __m128i m15 = _mm_set1_epi8(15), m8 = _mm_set1_epi8(8);
    int64_t b = 0;
    for (; b + 4 <= nb; b += 4)
        for (int k = 0; k < 4; k++) {
            __m128i v = _mm_loadu_si128((const __m128i *)(w + (b + k) * 16));
            __m128i lo = _mm_sub_epi8(_mm_and_si128(v, m15), m8);
            __m128i hi = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(v, 4), m15), m8);
            __m256i wv = _mm256_set_m128i(hi, lo);
            __m256i xv = _mm256_loadu_si256((const __m256i *)(x + (b + k) * 32));
            sums[b + k] = hsum8(dot32_i8(wv, xv));
        }
    if (b < nb) rko_blocksums_q4(w + b * 16, x + b * 32, nb - b, sums + b);
}

typedef struct {
    float *out;
    const void *w;
    const float *ws;
    const int8_t *qx;
    const float *xs;
    int64_t lo, hi, cols;
    int q4;
} mv_job;

static void *mv_worker(void *arg) {
    mv_job *j = arg;
    int64_t nb = j->cols / 32;
    int32_t *sums = malloc((size_t)nb * 4);
    for (int64_t i = j->lo; i < j->hi; i++) {
        if (j->q4)
            blocksums_q4_avx2((const uint8_t *)j->w + i * j->cols / 2, j->qx, nb, sums);
        else
            blocksums_q8_avx2((const int8_t *)j->w + i * j->cols, j->qx, nb, sums);
        j->out[i] = rko_qrow(sums, j->ws + i * nb, j->xs, nb);
    }
    free(sums);
    return NULL;
}

static void matvec_mt(float *out, const void *w, const float *ws, const float *x, int64_t rows, int64_t cols, int threads, int q4) {
    int64_t nb = cols / 32;
    int8_t *qx = malloc((size_t)cols);
    float *xs = malloc((size_t)nb * 4);
    rko_quantize8(x, cols, qx, xs);
    int64_t work = rows * cols / 65536;
    int workers = threads;
    if (work < workers) workers = (int)work;
    if (workers < 1) workers = 1;
    int64_t per = (rows + workers - 1) / workers;
    pthread_t tid[256];
    mv_job jobs[256];
    int n = 0;
    for (int64_t lo = 0; lo < rows && n < 256; lo += per, n++) {
        jobs[n] = (mv_job){out, w, ws, qx, xs, lo, lo + per < rows ? lo + per : rows, cols, q4};
        if (workers == 1)
            mv_worker(&jobs[n]);
        else
            pthread_create(&tid[n], NULL, mv_worker, &jobs[n]);
    }
    if (workers > 1)
        for (int i = 0; i < n; i++) pthread_join(tid[i], NULL);
    free(qx); free(xs);
}

void rko_matvec_q8_avx2_mt(float *out, const int8_t *w, const float *ws, const float *x, int64_t rows, int64_t cols, int threads) {
    matvec_mt(out, w, ws, x, rows, cols, threads, 0);
}
void rko_matvec_q4_avx2_mt(float *out, const uint8_t *w, const float *ws, const float *x, int64_t rows, int64_t cols, int threads) {
    matvec_mt(out, w, ws, x, rows, cols, threads, 1);
}

/* ------------------------------------------------------------------ */
/* Go math/rand/v2: PCG (128-bit LCG, DXSM output), Float64, IntN.       */
void rko_pcg_seed(rko_pcg *p, uint64_t s1, uint64_t s2) { p->hi = s1; p->lo = s2; }

uint64_t rko_pcg_uint64(rko_pcg *p) {
    const uint64_t mulHi = 2549297995355413924ull, mulLo = 4865540595714422341ull;
    const uint64_t incHi = 6364136223846793005ull, incLo = 1442695040888963407ull;
    unsigned __int128 prod = (unsigned __int128)p->lo * mulLo;
    uint64_t hi = (uint64_t)(prod >> 64), lo = (uint64_t)prod;
    hi += p->hi * mulLo + p->lo * mulHi;
    uint64_t lo2 = lo + incLo;
    uint64_t c = lo2 < lo;
    hi = hi + incHi + c;
    lo = lo2;
    p->lo = lo;
    p->hi = hi;
    const uint64_t cheapMul = 0xda942042e4dd58b5ull;
    hi ^= hi >> 32;
    hi *= cheapMul;
    hi ^= hi >> 48;
    hi *= (lo | 1);
    return hi;
}

double rko_rand_float64(rko_pcg *p) { return (double)(rko_pcg_uint64(p) << 11 >> 11) / 9007199254740992.0; }

int64_t rko_rand_intn(rko_pcg *p, int64_t n) {
    uint64_t un = (uint64_t)n;
    if ((un & (un - 1)) == 0) return (int64_t)(rko_pcg_uint64(p) & (un - 1));
    unsigned __int128 m = (unsigned __int128)rko_pcg_uint64(p) * un;
    uint64_t hi = (uint64_t)(m >> 64), lo = (uint64_t)m;
    if (lo < un) {
        uint64_t thresh = (0 - un) % un;
        while (lo < thresh) {
            m = (unsigned __int128)rko_pcg_uint64(p) * un;
            hi = (uint64_t)(m >> 64);
            lo = (uint64_t)m;
        }
    }
    return (int64_t)hi;
}

/* internal/num/num_test.go:351-369 transcendentalDigest's stream */
void rko_transcendental_words(uint64_t *out, int64_t steps) {
    rko_pcg rng;
    rko_pcg_seed(&rng, 9, 10);
    for (int64_t i = 0; i < steps; i++) {
        double f = rko_rand_float64(&rng);
        int64_t e = rko_rand_intn(&rng, 120) - 60;
        double x = ldexp(1 + f, (int)e);
        out[5 * i + 0] = d2u(rko_log(x));
        double g = rko_rand_float64(&rng);
        int64_t e2 = rko_rand_intn(&rng, 40);
        out[5 * i + 1] = d2u(rko_log1p(ldexp(g, -(int)e2)));
        double h = rko_rand_float64(&rng);
        out[5 * i + 2] = (uint64_t)f2u(rko_exp32((float)(h * 160 - 100)));
        double sc = rko_rand_float64(&rng);
        double s, c;
        rko_sincos((sc - 0.5) * 2e5, &s, &c);
        out[5 * i + 3] = d2u(s);
        out[5 * i + 4] = d2u(c);
    }
}

/* ------------------------------------------------------------------ */
/* Threads for the Q8 / Q4 products of rko_matvec (the forward, the head,
 * MoE): 0 (the default) runs the portable loops; n > 0 runs the AVX2 block
 * sums with rows over n threads, which give the same bits (the order is
 * per row, and block sums are exact), for model-size checks that must
 * finish in seconds. */
static int g_mv_threads = 0;
void rko_set_matvec_threads(int n) { g_mv_threads = n > 0 && rko_have_avx2() ? n : 0; }

/* internal/llm/model.go:170-188 Matrix.MulVec by storage type */
void rko_matvec(const rko_mat *m, float *out, const float *x) {
    if (g_mv_threads > 0 && (m->kind == RKO_Q8 || m->kind == RKO_Q4)) {
        if (m->kind == RKO_Q8)
            rko_matvec_q8_avx2_mt(out, m->q8, m->scales, x, m->rows, m->cols, g_mv_threads);
        else
            rko_matvec_q4_avx2_mt(out, m->q4, m->scales, x, m->rows, m->cols, g_mv_threads);
        return;
    }
    switch (m->kind) {
    case RKO_Q8: rko_matvec_q8(out, m->q8, m->scales, x, m->rows, m->cols); break;
    case RKO_Q4: rko_matvec_q4(out, m->q4, m->scales, x, m->rows, m->cols); break;
    case RKO_BF16: rko_matvec_bf16(out, m->bf16, x, m->rows, m->cols); break;
    default: rko_matvec32(out, m->f32, x, m->rows, m->cols); break;
    }
}

static int head_size(const rko_config *c) { return c->head_dim > 0 ? c->head_dim : c->dim / c->heads; }
static double theta_of(const rko_config *c) { return c->rope_theta > 0 ? c->rope_theta : 10000.0; }
static float eps_of(const rko_config *c) { return c->norm_eps > 0 ? (float)c->norm_eps : 1e-5f; }

/* internal/llm/model.go:428-441 NewRope (math.Log: fdlibm, as rko_log) */
void rko_rope_table(const rko_config *c, int32_t n, float *cos_t, float *sin_t) {
    int hs = head_size(c), half = hs / 2;
    double lt = rko_log(theta_of(c));
    for (int p = 0; p < half; p++) {
        double freq = rko_exp(((-lt) * (double)(2 * p)) / (double)hs);
        for (int pos = 0; pos < n; pos++) {
            double s, co;
            rko_sincos((double)pos * freq, &s, &co);
            cos_t[pos * half + p] = (float)co;
            sin_t[pos * half + p] = (float)s;
        }
    }
}

/* internal/llm/model.go:632-638 rmsNorm */
void rko_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps) {
    float ss = (rko_dot32(x, x, n) * rko_recip32((float)n)) + eps;
    float inv = rko_rsqrt32(ss);
    for (int64_t i = 0; i < n; i++) out[i] = w[i] * (inv * x[i]);
}

/* internal/llm/model.go:640-654 softmax */
void rko_softmax(float *x, int64_t n) {
    float mx = x[0];
    for (int64_t i = 1; i < n; i++) mx = rko_gomax(mx, x[i]);
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        x[i] = rko_exp32(x[i] - mx);
        sum += x[i];
    }
    float inv = rko_recip32(sum);
    for (int64_t i = 0; i < n; i++) x[i] = x[i] * inv;
}

/* internal/llm/model.go:570-588: one head's attention at a position, over
 * `positions` cached keys and values (kv_stride floats apart, the head's
 * slice at their start): scores float32(Dot32(q, k_t)·invSqrt), softmax, and
 * out[i] = Σ_t a_t·v_t[i] added in t order from +0. att holds the scores,
 * then the weights. */
void rko_attention_head(const float *qh, const float *keys, const float *vals, int64_t kv_stride, int hs,
                        int positions, float inv_sqrt, float *att, float *out) {
    for (int t = 0; t < positions; t++) att[t] = rko_dot32(qh, keys + (int64_t)t * kv_stride, hs) * inv_sqrt;
    rko_softmax(att, positions);
    for (int i = 0; i < hs; i++) out[i] = 0.0f;
    for (int t = 0; t < positions; t++) {
        const float *vt = vals + (int64_t)t * kv_stride;
        for (int i = 0; i < hs; i++) out[i] += att[t] * vt[i];
    }
}

/* internal/llm/model.go:657 silu */
float rko_silu(float v) { return v * rko_recip32(1.0f + rko_exp32(-v)); }

/* Elementwise evaluation for the device-math parity tests: fn 0 Recip32,
 * 1 Rsqrt32, 2 Exp32, 3 silu (internal/num/recip.go:38-93, num.go:76-97,
 * internal/llm/model.go:657). */
void rko_num_eval(int fn, const float *in, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float x = in[i];
        out[i] = fn == 0 ? rko_recip32(x) : fn == 1 ? rko_rsqrt32(x) : fn == 2 ? rko_exp32(x) : rko_silu(x);
    }
}

/* internal/llm/model.go:621-625 rotate */
static void rotate(float *v, int i, float co, float si) {
    float v0 = v[i], v1 = v[i + 1];
    v[i] = (v0 * co) - (v1 * si);
    v[i + 1] = (v0 * si) + (v1 * co);
}

/* internal/llm/model.go:529, gpustage.go:125: the scores' scale,
 * float32(1/math.Sqrt(float64(hs))): a float64 square root and division,
 * rounded once more to float32. */
float rko_inv_sqrt_head(int hs) { return (float)(1.0 / sqrt((double)hs)); }

/* internal/llm/model.go:522-613 Stage.Forward */
void rko_forward(const rko_config *c, const rko_layer *layers, int32_t nlayers, const float *cos_t, const float *sin_t,
                 float **keys, float **vals, int32_t ctx, float *x, int32_t pos, float *scratch) {
    int hs = head_size(c), qDim = c->heads * hs, kvDim = c->kv_heads * hs, dim = c->dim, hidden = c->hidden;
    int kvMul = c->heads / c->kv_heads, half = hs / 2;
    float invSqrt = rko_inv_sqrt_head(hs);
    float eps = eps_of(c);
    float *xb = scratch, *xb2 = xb + dim, *q = xb2 + dim, *k = q + qDim, *v = k + kvDim, *attOut = v + kvDim;
    float *hb = attOut + qDim, *hb2 = hb + hidden, *att = hb2 + hidden;
    (void)ctx;
    for (int li = 0; li < nlayers; li++) {
        const rko_layer *l = &layers[li];
        rko_rmsnorm(xb, x, l->rms_att, dim, eps);
        rko_matvec(&l->wq, q, xb);
        rko_matvec(&l->wk, k, xb);
        rko_matvec(&l->wv, v, xb);
        if (c->qkv_bias) {
            for (int i = 0; i < qDim; i++) q[i] += l->bq[i];
            for (int i = 0; i < kvDim; i++) k[i] += l->bk[i];
            for (int i = 0; i < kvDim; i++) v[i] += l->bv[i];
        }
        if (c->qk_norm) {
            for (int h = 0; h < qDim; h += hs) rko_rmsnorm(q + h, q + h, l->q_norm, hs, eps);
            for (int h = 0; h < kvDim; h += hs) rko_rmsnorm(k + h, k + h, l->k_norm, hs, eps);
        }
        const float *rc = cos_t + (int64_t)pos * half, *rs = sin_t + (int64_t)pos * half;
        for (int i = 0; i < qDim; i += 2) {
            int p = (i % hs) / 2;
            rotate(q, i, rc[p], rs[p]);
            if (i < kvDim) rotate(k, i, rc[p], rs[p]);
        }
        memcpy(keys[li] + (int64_t)pos * kvDim, k, (size_t)kvDim * 4);
        memcpy(vals[li] + (int64_t)pos * kvDim, v, (size_t)kvDim * 4);
        for (int h = 0; h < c->heads; h++) {
            int off = (h / kvMul) * hs;
            rko_attention_head(q + h * hs, keys[li] + off, vals[li] + off, kvDim, hs, pos + 1, invSqrt, att,
                               attOut + h * hs);
        }
        rko_matvec(&l->wo, xb2, attOut);
        for (int i = 0; i < dim; i++) x[i] += xb2[i];
        rko_rmsnorm(xb, x, l->rms_ffn, dim, eps);
        if (l->experts > 0) {
            /* the MoE feed-forward in place of SwiGLU, the same residual
             * (model.go:608-610): x = Canonical(x + y) */
            rko_moe_ffn(&l->router, l->ew1, l->ew2, l->ew3, l->experts, l->topk, xb, xb2, NULL, NULL);
            for (int i = 0; i < dim; i++) x[i] = rko_canonical(x[i] + xb2[i]);
            continue;
        }
        rko_matvec(&l->w1, hb, xb);
        rko_matvec(&l->w3, hb2, xb);
        for (int i = 0; i < hidden; i++) hb[i] = rko_silu(hb[i]) * hb2[i];
        rko_matvec(&l->w2, xb, hb);
        for (int i = 0; i < dim; i++) x[i] = rko_canonical(x[i] + xb[i]);
    }
}

/* internal/llm/model.go:216-231, 660-664 Embed via Matrix.Row */
void rko_embed(const rko_config *c, const rko_mat *t, int32_t token, float *x) {
    int64_t n = c->dim, nb = n / 32;
    switch (t->kind) {
    case RKO_Q8: rko_dequant8(x, t->q8 + token * n, t->scales + token * nb, n); break;
    case RKO_Q4: rko_dequant4(x, t->q4 + token * n / 2, t->scales + token * nb, n); break;
    case RKO_BF16:
        for (int64_t j = 0; j < n; j++) x[j] = rko_bf16(t->bf16[token * n + j]);
        break;
    default: memcpy(x, t->f32 + token * n, (size_t)n * 4); break;
    }
}

/* internal/llm/model.go:667-673 Head.Logits */
void rko_logits(const rko_config *c, const float *rms_final, const rko_mat *wcls, const float *x, float *logits) {
    float *xn = malloc((size_t)c->dim * 4);
    rko_rmsnorm(xn, x, rms_final, c->dim, eps_of(c));
    rko_matvec(wcls, logits, xn);
    free(xn);
}

/* internal/llm/sample.go:45-53 argmax: the first maximum wins */
int32_t rko_argmax(const float *v, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 0; i < n; i++)
        if (v[i] > v[best]) best = i;
    return (int32_t)best;
}

/* internal/llm/sample.go:11-16 NewSampler: a zero seed is replaced. */
uint64_t rko_sampler_seed(uint64_t seed) { return seed == 0 ? 0x9e3779b97f4a7c15ULL : seed; }

/* internal/llm/sample.go:18-24 next: xorshift64*, the top 24 bits of the
 * scrambled state over 2^24 (exact: k < 2^24 converts exactly and the
 * division is by a power of two). */
float rko_sampler_next(uint64_t *state) {
    uint64_t s = *state;
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    *state = s;
    return (float)((s * 0x2545f4914f6cdd1dULL) >> 40) / (float)(1 << 24);
}

/* internal/llm/sample.go:30-35: p_i = logit_i / T (a float32 division),
 * softmax (model.go:640-654). */
void rko_sample_probs(const float *logits, int64_t n, float temperature, float *p) {
    for (int64_t i = 0; i < n; i++) p[i] = logits[i] / temperature;
    rko_softmax(p, n);
}

/* internal/llm/sample.go:26-43 Sample: temperature <= 0 the greedy argmax;
 * else one draw r and the first i with r < cum, cum += p_i in order from
 * +0 (float32), else the last index. */
int32_t rko_sample(const float *logits, int64_t n, float temperature, uint64_t *state) {
    if (temperature <= 0) return rko_argmax(logits, n);
    float *p = malloc((size_t)n * 4);
    rko_sample_probs(logits, n, temperature, p);
    const float r = rko_sampler_next(state);
    float cum = 0.0f;
    int64_t pick = n - 1;
    for (int64_t i = 0; i < n; i++) {
        cum += p[i];
        if (r < cum) {
            pick = i;
            break;
        }
    }
    free(p);
    return (int32_t)pick;
}

/* ------------------------------------------------------------------ */
/* MoE feed-forward. The reference has no llama-family MoE; this build's
 * contract follows the dsv41 precedent (internal/llm/dsv41/ops.go:64-73
 * topK: stable, larger first, lower index wins ties; forward.go:355-411:
 * weight applied to the hidden activation, experts summed in ascending
 * expert index in float32):
 *   z = Q8 router · xn;  p = softmax(z) (model.go:640-654);
 *   sel = topK(p, k);  sum = p[sel0] + p[sel1] + ... (selection order);
 *   w_i = p[sel_i] · Recip32(sum);
 *   h_e = float32(w_e · float32(silu(W1_e xn) · W3_e xn));  o_e = W2_e h_e;
 *   y = 0; y += o_e for e ascending. */
/* Go's cmp.Compare on float32: NaN below every number, NaNs equal, -0 == +0. */
static int cmp_compare(float x, float y) {
    const int xn = x != x, yn = y != y;
    if (xn || yn) return xn && yn ? 0 : (xn ? -1 : 1);
    return x < y ? -1 : (x > y ? 1 : 0);
}
void rko_topk(const float *v, int32_t n, int32_t k, int32_t *idx) {
    /* internal/llm/dsv41/ops.go:67-74 topK: a stable sort by
     * cmp.Compare(v[b], v[a]), first k. As a selection: repeatedly the first
     * index whose value no remaining value compares above. */
    unsigned char *used = calloc((size_t)n, 1);
    for (int32_t s = 0; s < k; s++) {
        int32_t best = -1;
        for (int32_t i = 0; i < n; i++) {
            if (used[i]) continue;
            if (best < 0 || cmp_compare(v[i], v[best]) > 0) best = i;
        }
        used[best] = 1;
        idx[s] = best;
    }
    free(used);
}

void rko_moe_ffn(const rko_mat *router, const rko_mat *w1, const rko_mat *w2, const rko_mat *w3, int32_t experts,
                 int32_t topk, const float *xn, float *y, int32_t *sel_out, float *wsel_out) {
    int dim = router->cols, hidden = w1[0].rows;
    float *p = malloc((size_t)experts * 4);
    rko_matvec(router, p, xn);
    rko_softmax(p, experts);
    int32_t sel[64];
    float wsel[64];
    rko_topk(p, experts, topk, sel);
    float sum = 0.0f;
    for (int i = 0; i < topk; i++) sum += p[sel[i]];
    float inv = rko_recip32(sum);
    for (int i = 0; i < topk; i++) wsel[i] = p[sel[i]] * inv;
    float *g = malloc((size_t)hidden * 4), *u = malloc((size_t)hidden * 4), *o = malloc((size_t)dim * 4);
    for (int i = 0; i < dim; i++) y[i] = 0.0f;
    for (int e = 0; e < experts; e++) {
        int slot = -1;
        for (int i = 0; i < topk; i++)
            if (sel[i] == e) slot = i;
        if (slot < 0) continue;
        rko_matvec(&w1[e], g, xn);
        rko_matvec(&w3[e], u, xn);
        for (int i = 0; i < hidden; i++) g[i] = wsel[slot] * (rko_silu(g[i]) * u[i]);
        rko_matvec(&w2[e], o, g);
        for (int i = 0; i < dim; i++) y[i] += o[i];
    }
    if (sel_out)
        for (int i = 0; i < topk; i++) sel_out[i] = sel[i];
    if (wsel_out)
        for (int i = 0; i < topk; i++) wsel_out[i] = wsel[i];
    free(p); free(g); free(u); free(o);
}

/* ------------------------------------------------------------------ */
/* internal/sandbox/tensor.go:286-339 tenMatmul */
void rko_tensor_matmul_f32(const float *a, const float *b, float *c, int64_t m, int64_t k, int64_t n, int transposed) {
    int64_t stride = transposed ? 1 : n, step = transposed ? k : 1;
    for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++) {
            float acc = 0.0f;
            for (int64_t p = 0; p < k; p++) acc += a[i * k + p] * b[p * stride + j * step];
            c[i * n + j] = rko_canonical(acc);
        }
}
void rko_tensor_matmul_i8(const int8_t *a, const int8_t *b, int32_t *c, int64_t m, int64_t k, int64_t n, int transposed) {
    int64_t stride = transposed ? 1 : n, step = transposed ? k : 1;
    for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++) {
            uint32_t acc = 0; /* Go int32 arithmetic wraps */
            for (int64_t p = 0; p < k; p++) acc += (uint32_t)((int32_t)a[i * k + p] * (int32_t)b[p * stride + j * step]);
            c[i * n + j] = (int32_t)acc;
        }
}

/* internal/sandbox/tensor.go:445-461 tenQuantize (a true division) */
void rko_tensor_quantize(const float *a, int8_t *q, int64_t n, float k) {
    for (int64_t i = 0; i < n; i++) {
        float r = (float)rint((double)(a[i] / k));
        q[i] = (int8_t)(r != r ? 0 : (r > 127 ? 127 : (r < -127 ? -127 : r)));
    }
}

/* internal/sandbox/tensor.go:366-387 tenScale of an i32 tensor */
void rko_tensor_scale_i32(const int32_t *a, float *out, int64_t n, float k) {
    for (int64_t i = 0; i < n; i++) out[i] = rko_canonical((float)a[i] * k);
}
