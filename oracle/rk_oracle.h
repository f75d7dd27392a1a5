/*
 * rk_oracle.h — CPU restatement of rakkan-mesh's deterministic arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP backend
 * is compared against, bit for bit. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product library never links,
 * loads or calls it.
 *
 * Every function restates one function of the reference (Go) source; the
 * citation (path:line, relative to the reference repository) is beside each
 * definition in rk_oracle.c. Compiled with -O2 -ffp-contract=off
 * -fno-fast-math on x86-64 (SSE scalar float: every float32 operation rounds
 * once, as Go's explicit conversions demand).
 *
 * Each function is pinned, not just restated. The pins are the
 * reference's known answers and digests, its DeepSeek vectors, closed forms
 * and brute force, and exact-rational restatements that catch each
 * plausible slip (tests/test_oracle_*.py). Two areas are "parity unpinned"
 * against the reference:
 * - the MoE routing (rko_topk, rko_moe_ffn): the reference has no such
 *   model, so this build's own contract stands in for it;
 * - NaN payloads and Go's int8(NaN), which the parity inputs exclude.
 */
#ifndef RK_ORACLE_H
#define RK_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- internal/num/mx.go: DeepSeek-V4.1 block-scaled formats (rk_oracle_mx.c) ---- */
double rko_e4m3_value(uint8_t c);
uint8_t rko_encode_e4m3(float v);
void rko_encode_e4m3_n(const float *v, int64_t n, uint8_t *out);
float rko_decode_e8m0(uint8_t c);
float rko_decode_e2m1(uint8_t c);
uint8_t rko_encode_e2m1(float v);
float rko_pow2ceil(float t);
void rko_act_fp8(const float *x, int64_t n, uint8_t *codes, float *scales);
void rko_act_quant_inplace(float *x, int64_t n);
void rko_matvec_fp8(float *out, const uint8_t *w, const uint8_t *ws, const uint8_t *xc, const float *xs, int64_t rows,
                    int64_t cols, int bf16);
void rko_matvec_fp4(float *out, const uint8_t *w, const uint8_t *ws, const uint8_t *xc, const float *xs, int64_t rows,
                    int64_t cols, int bf16);
void rko_quantize_fp4(const float *x, int64_t n, int e4m3, uint8_t *packed, uint8_t *scales);
void rko_dequant_fp4(float *x, int64_t n, int e4m3, const uint8_t *packed, const uint8_t *scales);

/* ---- internal/num scalar functions ---- */
float rko_canonical(float v);
float rko_pow2(int k);
float rko_scale2(float v, int k);
float rko_recip32(float x);
float rko_rsqrt32(float x);
float rko_exp32(float x);
double rko_exp(double x);
double rko_log(double x);
double rko_log1p(double x);
float rko_log32(float x);
void rko_sincos(double x, double *s, double *c);
float rko_gomax(float x, float y);
uint16_t rko_to_bf16(float f);
float rko_bf16(uint16_t v);

/* ---- dot products and float matvecs ---- */
float rko_dot(const float *a, const float *b, int64_t n);
float rko_dot32(const float *a, const float *b, int64_t n);
float rko_dot_bf16(const uint16_t *w, const float *x, int64_t n);
void rko_matvec32(float *out, const float *w, const float *x, int64_t rows, int64_t cols);
void rko_matvec_bf16(float *out, const uint16_t *w, const float *x, int64_t rows, int64_t cols);

/* ---- Q8_0 / Q4_0 ---- */
void rko_quantize8(const float *w, int64_t n, int8_t *q, float *scales);
void rko_quantize4(const float *w, int64_t n, uint8_t *q, float *scales);
void rko_dequant8(float *dst, const int8_t *q, const float *scales, int64_t n);
void rko_dequant4(float *dst, const uint8_t *q, const float *scales, int64_t n);
void rko_blocksums_q8(const int8_t *w, const int8_t *x, int64_t nb, int32_t *sums);
void rko_blocksums_q4(const uint8_t *w, const int8_t *x, int64_t nb, int32_t *sums);
float rko_qrow(const int32_t *sums, const float *ws, const float *xs, int64_t nb);
void rko_matvec_q8(float *out, const int8_t *w, const float *ws, const float *x, int64_t rows, int64_t cols);
void rko_matvec_q4(float *out, const uint8_t *w, const float *ws, const float *x, int64_t rows, int64_t cols);
/* Q8 products of `tokens` inputs (rows of x), out[t*rows + r]: what the
 * per-token matvec gives each input (the batched-prefill contract). */
void rko_matmul_q8(float *out, const int8_t *w, const float *ws, const float *x, int64_t tokens, int64_t rows, int64_t cols);
void rko_matmul_q4(float *out, const uint8_t *w, const float *ws, const float *x, int64_t tokens, int64_t rows, int64_t cols);

/* CPU baseline: AVX2 block sums (the reference's blockSumsQ8AVX2 order of
 * work), rows split over threads. Bit-identical to rko_matvec_q8. */
void rko_matvec_q8_avx2_mt(float *out, const int8_t *w, const float *ws, const float *x, int64_t rows, int64_t cols, int threads);
void rko_matvec_q4_avx2_mt(float *out, const uint8_t *w, const float *ws, const float *x, int64_t rows, int64_t cols, int threads);
int rko_have_avx2(void);

/* ---- Go math/rand/v2 (PCG-DXSM) for the reference's own test streams ---- */
typedef struct { uint64_t hi, lo; } rko_pcg;
void rko_pcg_seed(rko_pcg *p, uint64_t s1, uint64_t s2);
uint64_t rko_pcg_uint64(rko_pcg *p);
double rko_rand_float64(rko_pcg *p);
int64_t rko_rand_intn(rko_pcg *p, int64_t n);
/* The stream TestTranscendentalsSameEverywhere hashes: 5 words per step. */
void rko_transcendental_words(uint64_t *out, int64_t steps);

/* ---- llm: the llama-family layer forward ---- */
enum { RKO_F32 = 0, RKO_BF16 = 1, RKO_Q8 = 2, RKO_Q4 = 3 };

typedef struct {
    int32_t kind, rows, cols, pad;
    const float *f32;
    const uint16_t *bf16;
    const int8_t *q8;
    const uint8_t *q4;
    const float *scales;
} rko_mat;

typedef struct {
    const float *rms_att, *rms_ffn, *bq, *bk, *bv, *q_norm, *k_norm;
    rko_mat wq, wk, wv, wo, w1, w2, w3;
    /* A mixture-of-experts feed-forward in place of w1/w2/w3 when experts
     * > 0: the router [experts][dim] and each expert's W1/W3 [hidden][dim]
     * and W2 [dim][hidden] (rko_moe_ffn), top `topk`. */
    int32_t experts, topk;
    rko_mat router;
    const rko_mat *ew1, *ew2, *ew3;
} rko_layer;

typedef struct {
    int32_t dim, hidden, layers, heads, kv_heads, vocab, seq_len, head_dim;
    double rope_theta, norm_eps;
    int32_t qkv_bias, qk_norm;
} rko_config;

void rko_matvec(const rko_mat *m, float *out, const float *x);
/* n > 0: rko_matvec's Q8 / Q4 products through the AVX2 block sums on n
 * threads (the same bits); 0: the portable loops. */
void rko_set_matvec_threads(int n);
void rko_rope_table(const rko_config *c, int32_t n, float *cos_t, float *sin_t);
void rko_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps);
void rko_softmax(float *x, int64_t n);
void rko_attention_head(const float *qh, const float *keys, const float *vals, int64_t kv_stride, int hs,
                        int positions, float inv_sqrt, float *att, float *out);
float rko_silu(float v);
float rko_inv_sqrt_head(int hs);
void rko_num_eval(int fn, const float *in, float *out, int64_t n);
/* One token through layers [0, nlayers) at position pos, x in place.
 * keys/vals: per layer [ctx][kvDim]. scratch: at least
 * 3*dim + 2*qDim + 2*kvDim + 2*hidden + ctx floats. */
void rko_forward(const rko_config *c, const rko_layer *layers, int32_t nlayers, const float *cos_t, const float *sin_t,
                 float **keys, float **vals, int32_t ctx, float *x, int32_t pos, float *scratch);
void rko_embed(const rko_config *c, const rko_mat *table, int32_t token, float *x);
void rko_logits(const rko_config *c, const float *rms_final, const rko_mat *wcls, const float *x, float *logits);
int32_t rko_argmax(const float *v, int64_t n);
uint64_t rko_sampler_seed(uint64_t seed);
float rko_sampler_next(uint64_t *state);
void rko_sample_probs(const float *logits, int64_t n, float temperature, float *p);
int32_t rko_sample(const float *logits, int64_t n, float temperature, uint64_t *state);

/* ---- MoE layer feed-forward (this build's contract; see rk_oracle.c) ---- */
void rko_topk(const float *v, int32_t n, int32_t k, int32_t *idx);
void rko_moe_ffn(const rko_mat *router, const rko_mat *w1, const rko_mat *w2, const rko_mat *w3, int32_t experts,
                 int32_t topk, const float *xn, float *y, int32_t *sel_out, float *wsel_out);

/* ---- rakkan_tensor_v1 host kernels ---- */
void rko_tensor_matmul_f32(const float *a, const float *b, float *c, int64_t m, int64_t k, int64_t n, int transposed);
void rko_tensor_matmul_i8(const int8_t *a, const int8_t *b, int32_t *c, int64_t m, int64_t k, int64_t n, int transposed);
void rko_tensor_quantize(const float *a, int8_t *q, int64_t n, float k);
void rko_tensor_scale_i32(const int32_t *a, float *out, int64_t n, float k);

#ifdef __cplusplus
}
#endif
#endif
