// rk_fused.h — the fused quantized products of a llama layer (rk_fused.hip):
// one kernel streams a product's weights and runs, before it, the input's
// RMSNorm and Q8 quantization (per workgroup, into LDS) and, after it, what
// the layer does next to each output row (bias, rotary embedding and cache
// store, SiLU gate, residual add, greedy argmax).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rk_kernels.h"

namespace rk {

enum : int32_t { kFmtQ8 = 0, kFmtQ4 = 1 };

// Where a product's input comes from.
enum : int32_t {
    kProGlobal = 0,  // already quantized (qx, xs, xsum), read from HBM/L2
    kProQuant = 1,   // f32 x, quantized by each workgroup into LDS
    kProNorm = 2,    // f32 x, RMSNorm'd with norm_w and quantized by each workgroup into LDS
};

// Widest input the RMSNorm prologue takes (x transposed in LDS beside the codes).
constexpr int kMaxNormProCols = 8192;

// What is done with each output row.
enum : int32_t {
    kEpStore = 0,     // out = W·x (+ bias)
    kEpAdd = 1,       // out += W·x                         (residual, internal/llm/model.go:596-598)
    kEpAddCanon = 2,  // out = Canonical(out + W·x)          (model.go:608-610)
    kEpQKV = 3,       // [Wq;Wk;Wv]·x + bias, RoPE on q and k pairs, k and v into the caches at the position
    kEpSilu = 4,      // rows interleaved W1,W3: h = silu(W1·x)·(W3·x)  (model.go:603-605)
    kEpLogits = 5,    // logits = W·x and their greedy argmax; the position advances
};

// Largest input width the LDS prologues take (f32 staging + codes + scales).
constexpr int kMaxLdsCols = 16384;

// Device control words of a stage: the generation state lives on the GPU so
// that one recorded token replays unchanged at every position.
enum : int { kCtlPos = 0, kCtlPrompt = 1, kCtlWords = 4 };

// 64-bit words of a hand-off between the workgroups of one launch
// (launch_att_values_wo): producers done, waiting workgroups started, a
// waiter gave up, then one flag word per XCD, 128 bytes apart. Zero when
// allocated; never reset.
enum : int {
    kSyncDone = 0,
    kSyncArrive = 1,
    kSyncError = 2,
    kSyncFlag = 16,
    kSyncFlagStride = 16,
    kSyncWords = kSyncFlag + 8 * kSyncFlagStride
};
// Longest wait of a waiting workgroup: 20 ms of the 100 MHz real-time clock.
constexpr unsigned long long kSyncTimeout = 2000000ull;

// The classifier's greedy argmax is folded into kArgmaxSlots 64-bit keys
// (atomicMax, spread over slots so the workgroups do not queue on one
// address); the key of logit v at row i orders by value, then by lower row.
constexpr int kArgmaxSlots = 16;

// LDS a workgroup may use on gfx950 (kernels asking more than 64 KiB set
// their limit first).
constexpr size_t kMaxLdsBytes = 160 * 1024;

// Largest context the attention-values kernel keeps its weights for.
int att_values_max_ctx();

// Largest vector a single-workgroup norm keeps in LDS.
constexpr int kMaxNormCols = 12288;


struct FusedArgs {
    MatSeg seg[3];        // Q/K/V, or W1/W3 (interleaved row by row), or one matrix
    int32_t nseg;
    int32_t cols;         // input width (multiple of 32)
    int32_t rows;         // logical output rows (all segments)
    int32_t rows_per_wg;  // set by the launcher
    int32_t row_base;     // kEpQKV: logical index of row 0 (a Q/K/V split over two launches)
    // input
    const float *x;       // f32 input (kProQuant, kProNorm)
    const float *norm_w;  // kProNorm: RMSNorm weights (internal/llm/model.go:632-638)
    float recip_n, norm_eps;
    const int8_t *qx;     // quantized input (kProGlobal)
    const float *xs;
    const int32_t *xsum;
    // epilogue
    const float *bias;    // per logical row, or null
    int32_t *ctl;         // control words (kCtl*)
    const float *cos_t, *sin_t;  // rotary table [ctx][hs/2]
    int32_t hs, qdim, kvdim;
    float *kcache, *vcache;      // this layer's [ctx][kvdim]
    unsigned long long *amax;    // logits: kArgmaxSlots keys (zero before the product)
    int32_t gate;                // logits: 1 = skip the product at prompt positions before the last
    int8_t *qx_out;              // kEpSilu: h quantized for the next product (or null)
    float *xs_out;
    int32_t *xsum_out;
    // LDS layout (bytes), set by the launcher
    int32_t lds_xs, lds_xsum, lds_norm, lds_res, lds_ep, lds_bytes;
};

// Whether the LDS prologue (kProQuant) takes an input of `cols`.
bool fused_fits(int pro, int cols);

// Enqueues one fused product. fmt: kFmtQ8/kFmtQ4; returns false when the
// shape does not fit the kernel (cols beyond kMaxLdsCols with an LDS
// prologue, or too many workgroups for the argmax partials). Widths with a
// static-schedule instance (rk_stream.hip) run there, the others in
// fused_kernel; the results are the same.
bool launch_fused(int fmt, int pro, int epi, FusedArgs a, int cu, hipStream_t s);

// The static-schedule products (rk_stream.hip): false when no instance
// takes (fmt, pro, epi) at this width and shape.
bool launch_stream(int fmt, int pro, int epi, FusedArgs a, int cu, hipStream_t s);
// Whether an instance exists for (fmt, pro, epi) at width cols.
bool stream_has(int fmt, int pro, int epi, int cols);

// A batch of consecutive positions for the attention kernels: token z sits
// at pos0 + z and attends to positions 0..pos0+z; its rows are z·stride
// floats into the q, scores and output buffers. Used when ctl is null.
// Independent sequences: with `pos` set, token z is sequence z, at position
// pos[z] (device memory), attending to its own cache, cache_stride floats
// after sequence z-1's.
struct AttBatch {
    int32_t pos0 = 0, tokens = 1;
    int64_t q_stride = 0, att_stride = 0, out_stride = 0;
    const int32_t *pos = nullptr;
    int64_t cache_stride = 0;
};

// Position of token z of an attention launch: the stage's (ctl), the
// sequence's own (bt.pos), or z after the batch's first.
__device__ __forceinline__ int att_position(const int32_t *ctl, const AttBatch &bt, int z) {
    return ctl ? ctl[kCtlPos] : (bt.pos ? bt.pos[z] : bt.pos0 + z);
}

// Attention of one position over a stage's cache (internal/llm/model.go:
// 575-591), position and length read from ctl (or, ctl null, a batch):
// scores, then softmax and the weighted values (f32 out).
void launch_att_scores(const float *q, const float *keys, float *att, int32_t att_stride, const int32_t *ctl,
                       const AttBatch &bt, int ctx, int heads, int kv_heads, int hs, int kv_dim, float inv_sqrt,
                       hipStream_t s);
// The same scores with QK-norm and RoPE of the position's raw q and k
// (launch_qknorm_rope's steps) folded in, k and v stored into the caches:
// for a decode step (ctl) or independent sequences (bt.pos); false (nothing
// launched) for other batches or shapes.
bool launch_att_scores_qkn(const float *q_raw, const float *k_raw, const float *v_raw, const float *q_norm,
                           const float *k_norm, float recip_hs, float eps, const float *cos_t, const float *sin_t,
                           float *keys, float *vals, float *att, int32_t att_stride, const int32_t *ctl,
                           const AttBatch &bt, int ctx, int heads, int kv_heads, int hs, int kv_dim, float inv_sqrt,
                           hipStream_t s);
// Batches up to 1024 positions (head size a multiple of 32) run a group of
// tokens per workgroup (rk_attn_batch.hip); the results are the same.
bool att_group_fits(const AttBatch &bt, int hs, int kv_dim);
void launch_att_scores_group(const float *q, const float *keys, float *att, int32_t att_stride, const AttBatch &bt,
                             int heads, int kv_heads, int kv_dim, float inv_sqrt, hipStream_t s);
void launch_att_values_group(const float *att, int32_t att_stride, const float *vals, float *out, const AttBatch &bt,
                             int heads, int kv_heads, int hs, int kv_dim, int8_t *qx, float *xs, int32_t *xsum,
                             hipStream_t s, int cu = 0);
// With qx non-null (head size a multiple of 32), the output is also
// quantized (Q8_0 blocks of the next product's input).
void launch_att_values(const float *att, int32_t att_stride, const float *vals, float *out, const int32_t *ctl,
                       const AttBatch &bt, int ctx, int heads, int kv_heads, int hs, int kv_dim, int8_t *qx,
                       float *xs, int32_t *xsum, hipStream_t s, int cu = 0);
// The values of a decode step (position in ctl) and the Wo product that
// reads their Q8_0 form, x[r] += Wo_r·attn, in one launch: the values
// workgroups as launch_att_values (contexts up to 1024), then workgroups of
// Wo rows (16 for contexts up to 256, else 32) whose codes are requested at
// the launch's start and wait for the last values workgroup through `sync`
// (kSyncWords words). The results are those of the two launches, bit for
// bit. False (nothing launched) when the shapes are not the ones it takes:
// a Q8_0 Wo of 3073..4096 columns (heads·hs, hs a multiple of 32), rows a
// multiple of the workgroup's. With qk (a QK-norm layer's raw q, k and v,
// contexts up to 256, hs = 128, else false) the launch also forms the
// scores (launch_att_scores_qkn's work, the same bits), so it is the whole
// attention of the step after the QKV product.
struct QknIn {
    const float *q_raw, *k_raw, *v_raw, *q_norm, *k_norm, *cos_t, *sin_t;
    float *keys, *vals;  // the caches, where the position's k and v go
    float recip_hs, eps, inv_sqrt;
};
bool launch_att_values_wo(const float *att, int32_t att_stride, const float *vals, float *out, const int32_t *ctl,
                          int ctx, int heads, int kv_heads, int hs, int kv_dim, int8_t *qx, float *xs, int32_t *xsum,
                          const uint8_t *wo_w, const float *wo_ws, int64_t wo_rows, int64_t wo_cols, float *x,
                          unsigned long long *sync, hipStream_t s, const QknIn *qk = nullptr);
// QK-norm (Qwen3) and RoPE of raw q and k heads, k and v into the caches, at
// the position in ctl (or, ctl null, for `tokens` rows at pos0, pos0+1, ...;
// or, seq_pos set, row z at seq_pos[z] in caches cache_stride floats apart).
void launch_qknorm_rope(float *q, const float *k, const float *v, const float *q_norm, const float *k_norm,
                        float recip_hs, float eps, const float *cos_t, const float *sin_t, const int32_t *ctl,
                        int32_t pos0, int tokens, float *kcache, float *vcache, int heads, int kv_heads, int hs,
                        hipStream_t s, const int32_t *seq_pos = nullptr, int64_t cache_stride = 0);
// x = the embedding row of tokens[ctl[kCtlPos]] (Q8_0 or Q4_0 table), and
// RMSNorm(x) with norm_w quantized into qx/xs/xsum (one workgroup;
// dim <= kMaxNormCols).
void launch_embed_norm(const uint8_t *w, const float *scales, bool q4, const int32_t *tokens, const int32_t *ctl,
                       int dim, float *x, const float *norm_w, float recip_n, float eps, int8_t *qx, float *xs,
                       int32_t *xsum, hipStream_t s);
// Embedding rows of tokens[pos0..pos0+n) (Q8_0 or Q4_0 table) into x
// [n][dim], as embed_norm gives them one position at a time; with seq_pos,
// row z is sequence z's token at its position, tokens[z·tok_stride +
// seq_pos[z]].
void launch_embed_rows(const uint8_t *w, const float *scales, bool q4, const int32_t *tokens, int32_t pos0, int n,
                       int dim, float *x, hipStream_t s, int64_t tok_stride = 0, const int32_t *seq_pos = nullptr);
// Independent sequences' greedy step: the argmax of each of `seqs` logits
// rows ([seqs][vocab]) becomes that sequence's token at pos[z]+1 (past its
// prompt), and pos[z] advances.
void launch_seqs_advance(const float *logits, int64_t vocab, int seqs, int32_t *pos, const int32_t *prompt,
                         int32_t *tokens, int64_t tok_stride, int32_t tokens_len, hipStream_t s);
// The seeded sampler's step (internal/llm/sample.go:26-43) for `seqs`
// logits rows [seqs][vocab]: sequence z picks its token at pos[z]+1 when
// that position is past its prompt (the argmax when temps[z] <= 0, else a
// draw from softmax(logits/T) with the xorshift64* state states[z], which
// advances once a draw), and pos[z] advances. terms: [seqs][stride] floats
// (sample_terms_stride), part: [seqs][sample_parts()] floats, both scratch.
struct SampleArgs {
    const float *logits;
    int64_t vocab;
    int seqs;
    int32_t *pos;
    const int32_t *prompt;
    int32_t *tokens;
    int64_t tok_stride;
    int32_t tokens_len;
    const float *temps;
    uint64_t *states;
    float *terms, *part;
    unsigned long long *amax;  // one sequence: the classifier's argmax keys, cleared (else null)
};
int64_t sample_terms_stride(int64_t vocab);
int sample_parts();
void launch_sample(const SampleArgs &a, hipStream_t s);
// The greedy argmax's end (internal/llm/sample.go:45-53): folds the
// classifier's argmax keys into the next token at position+1 (when the
// position's logits were computed), clears them, and advances the position.
void launch_advance(int32_t *ctl, unsigned long long *amax, int32_t *tokens, int32_t tokens_len, hipStream_t s);
// RMSNorm(x) with norm_w quantized into qx/xs/xsum: `tokens` rows of
// [tokens][n] at once (one workgroup each; n <= kMaxNormCols).
void launch_norm_quant(const float *x, int n, const float *norm_w, float recip_n, float eps, int8_t *qx, float *xs,
                       int32_t *xsum, hipStream_t s, int tokens = 1);

}  // namespace rk
