/*
 * rk.h — C-ABI of the MI355X (gfx950) backend for rakkan-mesh's quantized
 * matrix-vector hot path: librkhip.so.
 *
 * The entry points replace the bodies of the Go API in internal/gpu (the
 * Vulkan backend) one for one; each declaration cites the Go interface it
 * stands in for (paths relative to the rakkan-mesh repository). A cgo shim in
 * internal/gpu keeps the exported Go names and signatures and calls these.
 *
 * Conventions:
 *   - Every function returns an int status (RK_OK or a negative RK_ERR_*),
 *     except the few documented getters. Nothing aborts the process; the text
 *     of the last error on a device is rk_last_error(dev).
 *   - Host buffers are owned by the caller and only read or written during
 *     the call. Handles are opaque; the caller frees them, before
 *     rk_device_close (as internal/gpu/device.go:344-378 requires).
 *   - A device is safe for concurrent use; calls that touch it run one at a
 *     time (internal/gpu/device.go:202-203), on one HIP stream.
 *   - Results are bit-identical to the reference's CPU path (internal/num):
 *     integer block sums, then the fixed-order float32 combine of
 *     internal/num/quant.go:14-19, 158-164.
 */
#ifndef RK_H
#define RK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    RK_OK = 0,
    RK_ERR_ARGS = -1,        /* bad handle, shape, type or offset */
    RK_ERR_OOM = -2,         /* device memory exhausted */
    RK_ERR_HIP = -3,         /* a HIP runtime call failed */
    RK_ERR_UNSUPPORTED = -4, /* a format this build does not run */
    RK_ERR_NO_DEVICE = -5,   /* no usable GPU */
};

/* Matrix storage formats (internal/gpu/device.go:562-585 Format). */
enum {
    RK_F32 = 0,
    RK_BF16 = 1,
    RK_Q8 = 2, /* int8 codes [rows][cols], float32 scales [rows][cols/32] */
    RK_Q4 = 3, /* nibbles [rows][cols/2] (low: j, high: j+16 of a block), scales as Q8 */
    RK_FP8 = 4, /* E4M3 codes [rows][cols], E8M0 scale bytes [ceil(rows/32)][cols/32] */
    RK_FP4 = 5, /* E2M1 codes [rows][cols/2] (low nibble: even element), E8M0 bytes [rows][cols/32] */
};

typedef struct rk_device rk_device;
typedef struct rk_matrix rk_matrix;

typedef struct {
    int32_t index;
    char name[64];
    char arch[32];       /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int64_t memory;      /* device-local bytes */
    int32_t compute_units;
    int32_t exact;       /* 1: IEEE f32 with denormals kept, round to nearest even */
    int32_t integrated;  /* 1: an integrated GPU (device.go Info.Type "integrated"), 0: discrete */
} rk_device_info;

/* internal/gpu/device.go:125-183 Devices (count, then rk_device_info per index). */
int rk_device_count(int32_t *count);
int rk_device_info_get(int32_t index, rk_device_info *info);

/* internal/gpu/device.go:238-279 Open; :344-378 Close. */
int rk_device_open(int32_t index, rk_device **out);
int rk_device_close(rk_device *dev);

/* internal/gpu/device.go Device.Used: bytes of matrices, vectors and arenas
 * held. Returns -1 for a null device. */
int64_t rk_used_bytes(rk_device *dev);

/* Text of the last error on dev (or of the last failed open when dev is
 * NULL); valid until the next call on the device. */
const char *rk_last_error(rk_device *dev);

/* internal/gpu/device.go:587-700 Upload. w: F32 float[rows*cols], BF16
 * uint16[rows*cols], Q8 int8[rows*cols], Q4 uint8[rows*cols/2]; scales:
 * float[rows*cols/32] for Q8/Q4, NULL otherwise. Shape limits as the
 * reference: cols <= 2^18, rows <= 2^24, cols % 32 == 0 for Q8/Q4. The
 * device layout is this build's own (the reference layout is repacked). */
int rk_matrix_upload(rk_device *dev, int32_t kind, int64_t rows, int64_t cols, const void *w, const float *scales,
                     rk_matrix **out);

/* internal/gpu/device.go:562-585, 587-700 Upload of Format{FP8 | FP4, E8M0}
 * (DeepSeek-V4.1's block-scaled matrices): kind RK_FP8 or RK_FP4, codes and
 * E8M0 scale bytes laid out as the enum above says. E4M3 NaN codes (0x7f,
 * 0xff) are refused ("gpu: NaN in E4M3 weights"), as num.ValidE4M3 is
 * checked there. Their products (rk_matvecs, rk_matvecs_device,
 * rk_batch_matvecs) quantize the input to E4M3 with a power-of-two scale
 * per 32 (num.QuantizeActFP8) and return num.MatVecFP8 / MatVecFP4 bit for
 * bit, rounded to bfloat16 (internal/num/mx.go:282-334). */
int rk_matrix_upload_mx(rk_device *dev, int32_t kind, int64_t rows, int64_t cols, const uint8_t *w,
                        const uint8_t *e8m0, rk_matrix **out);

/* internal/gpu/device.go:575-581, 609-618, 704-723 Upload of
 * Format{FP4Chunks, E8M0Chunks, AlignRows} (stacked experts, uploaded piece
 * by piece and never gathered on the host whole; internal/llm/dsv41/gpu.go:
 * 177-184): the codes as n_w pieces w[i] of w_len[i] bytes and the E8M0
 * scales as n_s pieces, each list read as one run of bytes, laid out as
 * rk_matrix_upload_mx's. align_rows > 0: rows must be a whole number of
 * runs of that many rows (and, for E4M3, a multiple of 32), else
 * "gpu: rows not a whole number of aligned runs". The matrix is one device
 * allocation, so the runs are whole by construction. The same checks and
 * messages as rk_matrix_upload_mx, in the reference's order. */
int rk_matrix_upload_mx_chunks(rk_device *dev, int32_t kind, int64_t rows, int64_t cols, int32_t n_w,
                               const uint8_t *const *w, const int64_t *w_len, int32_t n_s,
                               const uint8_t *const *e8m0, const int64_t *s_len, int32_t align_rows,
                               rk_matrix **out);

/* internal/gpu/device.go:548 Matrix.unrounded: raw != 0 leaves an E4M3 /
 * E2M1 matrix's products in float32 (num.MatVecFP8Unrounded), for checks
 * where bfloat16 would hide the last bits. */
int rk_matrix_set_raw(rk_matrix *m, int32_t raw);

/* internal/gpu/device.go:733-738 Matrix.Free. */
int rk_matrix_free(rk_matrix *m);

/* internal/gpu/device.go:727 Matrix.Bytes (-1 for NULL). */
int64_t rk_matrix_bytes(const rk_matrix *m);

/* internal/gpu/device.go:769-793 MulVecs: outs[i] = ms[i]·x for n matrices
 * on one device sharing cols; x (cols floats) and outs are host buffers. The
 * input is quantized once for the Q8/Q4 matrices (internal/gpu/batch.go:214-269).
 * Blocking, like the reference's submit-and-wait. */
int rk_matvecs(rk_device *dev, int32_t n, rk_matrix *const *ms, float *const *outs, const float *x, int64_t cols);

/* The same products with device-resident x and outputs, enqueued on the
 * HIP stream `stream` (NULL: the device's own) without waiting. For callers
 * that keep activations in HBM (a stage executor, benchmarks). */
int rk_matvecs_device(rk_device *dev, int32_t n, rk_matrix *const *ms, float *const *d_outs, const float *d_x,
                      int64_t cols, void *stream);

/* ---- Batched products (prompt prefill) ----
 * No reference counterpart: the reference runs a prompt one token at a time
 * (internal/llm/model.go:504-518), each token's products through MulVecs
 * (internal/gpu/device.go:769-793). For each of `tokens` inputs
 * x_t = x + t·cols: outs[i] + t·rows_i receives ms[i]·x_t, bit for bit what
 * rk_matvecs gives for x_t alone. The block sums run on int8 MFMA. Host
 * buffers, blocking. */
int rk_matmul_t(rk_device *dev, int32_t n, rk_matrix *const *ms, float *const *outs, const float *x, int64_t cols,
                int32_t tokens);
/* The same with device-resident x ([tokens][cols]) and outputs
 * ([tokens][rows_i]), enqueued on `stream` (NULL: the device's own). */
int rk_matmul_t_device(rk_device *dev, int32_t n, rk_matrix *const *ms, float *const *d_outs, const float *d_x,
                       int64_t cols, int32_t tokens, void *stream);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc): rk_matmul_t_device's products, bit for bit, with the tokens'
 * quantized inputs in a static device array of the library (about 20 MiB
 * per GPU, held until the process ends) instead of a scratch grown with
 * hipMalloc. It allocates nothing. tokens·cols must not pass 2^24 (16,777,216
 * codes, e.g. 512 tokens of 32768 columns); a larger call returns
 * RK_ERR_ARGS before enqueuing anything. Every call on a device shares the
 * array: calls that overlap on one device (on streams without an order
 * between them) race on it, so the caller orders them. */
int rk_matmul_t_device_noalloc(rk_device *dev, int32_t n, rk_matrix *const *ms, float *const *d_outs,
                               const float *d_x, int64_t cols, int32_t tokens, void *stream);

/* ---- Arenas, vectors and batches (internal/gpu/batch.go) ----
 * An arena is device memory of 32-bit words holding a computation's
 * activations, caches and tables; batch operations address it by word
 * offsets, as the Go API does. Every span an operation names is checked
 * against its arena or vectors; a bad one latches RK_ERR_ARGS. */
typedef struct rk_arena rk_arena;
typedef struct rk_vectors rk_vectors;
typedef struct rk_batch rk_batch;

/* internal/gpu/batch.go:22-49 NewArena: `words` of device memory and pinned
 * staging for `staging_words` moved per submission. */
int rk_arena_new(rk_device *dev, int64_t words, int64_t staging_words, rk_arena **out);
/* internal/gpu/batch.go:51-55 SetQuantScratch: reserves room for a quantized
 * input: at qx_off cols/4 words (Q8_0 codes, four a word) or cols words
 * (E4M3 values), at xs_off cols/32 words (block scales). Products keep their
 * quantized input in the arena's own 16-byte-aligned scratch (read as
 * 128-bit vectors) and leave the reserved words as they were; rk_batch_quantize
 * and rk_batch_quantize_fp8 write their result there, in the reference's
 * layout. */
int rk_arena_set_quant_scratch(rk_arena *a, int64_t qx_off, int64_t xs_off);
/* internal/gpu/batch.go:57-58 Bytes. */
int64_t rk_arena_bytes(const rk_arena *a);
/* internal/gpu/batch.go:60-71 Free. */
int rk_arena_free(rk_arena *a);
/* Device address of word `off`, for rk_matvecs_device and other callers that
 * pass device pointers. No reference counterpart (Vulkan never exposes one). */
int rk_arena_device_ptr(rk_arena *a, int64_t off, void **dptr);

/* internal/gpu/batch.go:82-109 UploadVectors / Vectors.Free: a layer's norm
 * weights and biases, read by rmsnorm and addvec. */
int rk_vectors_upload(rk_device *dev, const float *v, int64_t n, rk_vectors **out);
int rk_vectors_free(rk_vectors *v);

/* internal/gpu/batch.go:126-134 Begin: holds the device until submit.
 * Operations return the batch's first error so far (RK_OK if none); after an
 * error they do nothing, and submit returns it (batch.go:136-147). */
int rk_batch_begin(rk_arena *a, rk_batch **out);
/* internal/gpu/batch.go:149-159 Write: copies n floats to word off. */
int rk_batch_write(rk_batch *b, int64_t off, const float *data, int64_t n);
/* internal/gpu/batch.go:161-171 Read: n words at off into dst on submit. */
int rk_batch_read(rk_batch *b, int64_t off, float *dst, int64_t n);
/* internal/gpu/batch.go:212-269 MatVecs: ms[i]·x into word out_offs[i], x
 * at in_off, quantized once (Q8/Q4 need the arena's quant scratch). */
int rk_batch_matvecs(rk_batch *b, int32_t n, rk_matrix *const *ms, const int64_t *out_offs, int64_t in_off);
/* internal/gpu/batch.go:277-280 Quantize: n floats at in to Q8_0: codes four
 * a word (code j in byte j) at qx_off, block scales at xs_off. */
int rk_batch_quantize(rk_batch *b, int64_t in, int64_t n);
/* internal/gpu/dsbatch.go:142-172 ExpertMatVecs: m holds E2M1 experts of
 * per_expert rows each (a multiple of 8 here; RK_ERR_UNSUPPORTED otherwise);
 * slot k (of slots) multiplies expert ids[k] (uint32 words at arena word
 * `ids`; an id past the last expert is skipped) by input k / div (div 0:
 * one input for all) at word in + (k/div)·in_stride into out + k·out_stride.
 * The inputs are quantized into the arena's quantize scratch, which must be
 * set and hold them (inputs·cols <= 2^18). */
int rk_batch_expert_matvecs(rk_batch *b, rk_matrix *m, int64_t per_expert, int64_t ids, int32_t slots, int64_t in,
                            int64_t in_stride, int32_t div, int64_t out, int64_t out_stride);

/* internal/gpu/dsbatch.go:174-210 MatVecsBatch: m times n inputs at words
 * in + j·in_stride into out + j·out_stride, each output MatVecs' bits (one
 * product an input here; the weights are read once an input). */
int rk_batch_matvecs_batch(rk_batch *b, rk_matrix *m, int64_t out, int64_t out_stride, int64_t in, int64_t in_stride,
                           int32_t n);

/* internal/gpu/dsbatch.go:60-74 ActQuantInPlace (num.ActQuantInPlace: each
 * value its E4M3 rounding times its block's power-of-two scale, in
 * bfloat16; n a multiple of 32) and FP4QuantInPlace (num.FP4QuantInPlace:
 * E2M1 codes with E4M3 scales per 16 if e4m3, else E8M0 per 32, dequantized
 * to bfloat16) of n floats at word off, in place. */
int rk_batch_act_quant_inplace(rk_batch *b, int64_t off, int64_t n);
int rk_batch_fp4_quant_inplace(rk_batch *b, int64_t off, int64_t n, int32_t e4m3);

/* internal/gpu/batch.go:271-275 QuantizeFP8: n floats at word `in` to E4M3
 * with block scales, as num.QuantizeActFP8: the codes' values, unscaled, as n
 * float32 words at qx_off (internal/gpu/mx.go:146-172), the scales at
 * xs_off. A NaN code (an input block holding an infinity or NaN) reads as
 * NaN, num.ActFP8.Vals' value; the reference's Vulkan kernel gives ±480. */
int rk_batch_quantize_fp8(rk_batch *b, int64_t in, int64_t n);

/* internal/gpu/batch.go:282-287 RMSNorm: segs segments of n floats at in
 * (stride apart) into out: out = w·(Rsqrt32(Dot32(x,x)·recip_n + eps)·x). */
int rk_batch_rmsnorm(rk_batch *b, rk_vectors *vecs, int64_t in, int64_t out, int64_t w, int32_t n, int32_t segs,
                     int64_t stride, float recip_n, float eps);
/* internal/gpu/batch.go:289-292 AddVec: n floats at word v of vecs added to out. */
int rk_batch_addvec(rk_batch *b, rk_vectors *vecs, int64_t out, int64_t v, int64_t n);
/* internal/gpu/batch.go:294-298 Rope: adjacent pairs of q (q_dim) and k
 * (kv_dim) with the position's cos and sin rows (head_size/2 each). */
int rk_batch_rope(rk_batch *b, int64_t q, int64_t k, int32_t q_dim, int32_t kv_dim, int32_t head_size, int64_t cos,
                  int64_t sin);
/* internal/gpu/batch.go:300-303 Copy: n words. */
int rk_batch_copy(rk_batch *b, int64_t src, int64_t dst, int64_t n);
/* internal/gpu/batch.go:305-316 Attention for one position: scores of q
 * against keys (positions rows, kv_dim apart) into att (heads rows,
 * att_stride apart), softmax, and the values weighted into out. */
int rk_batch_attention(rk_batch *b, int64_t q, int64_t keys, int64_t vals, int64_t att, int64_t att_stride, int64_t out,
                       int32_t positions, int32_t heads, int32_t kv_heads, int32_t head_size, int32_t kv_dim,
                       float inv_sqrt);
/* internal/gpu/batch.go:318-326 Residual: x += y, NaNs canonical if asked. */
int rk_batch_residual(rk_batch *b, int64_t x, int64_t y, int64_t n, int32_t canonical);
/* internal/gpu/batch.go:328-331 SiluMul: a = silu(a)·b. */
int rk_batch_silumul(rk_batch *b, int64_t a, int64_t b_off, int64_t n);
/* internal/gpu/batch.go:333-349 Submit: waits, delivers the reads, releases
 * the device and frees the batch; returns the first error. */
int rk_batch_submit(rk_batch *b);

/* ---- Graphs ----
 * Records the work that device-pointer calls (rk_matvecs_device with a NULL
 * stream, and the other *_device entry points) enqueue on the device's
 * stream between rk_graph_begin and rk_graph_end into a HIP graph, which
 * rk_graph_launch replays: the same kernels on the same buffers, without
 * the per-call host cost. No reference counterpart: the reference
 * re-records its Vulkan command buffer for every submission
 * (internal/gpu/batch.go:126-134). Only one thread may use the device while
 * it records; batches (which wait) cannot be recorded. */
typedef struct rk_graph rk_graph;
int rk_graph_begin(rk_device *dev);
int rk_graph_end(rk_device *dev, rk_graph **out);
/* Enqueues `times` replays on the device stream and waits for them. */
int rk_graph_launch(rk_graph *g, int32_t times);
/* rk_graph_launch with the replays bracketed by two events on the device
 * stream: *ms is the device time from the first replay's start to the last
 * one's end (the host's enqueue cost is not in it). */
int rk_graph_launch_timed(rk_graph *g, int32_t times, float *ms);
int rk_graph_free(rk_graph *g);

/* ---- Stages: a run of llama-family layers resident on one device ----
 * internal/llm/gpustage.go (gpuStage): the layers' products, attention and
 * caches run on the device; Stage.ForwardMany (internal/llm/model.go:
 * 488-502) hands it token activations. This build fuses the stage: each
 * product's kernel also does the RMSNorm and Q8 quantization of its input
 * and the step after it (bias, RoPE and the cache store, SiLU·mul, the
 * residual add), and every position-dependent value (position, length,
 * tokens) is read from device memory, so one token is recorded once as a
 * HIP graph and replayed at every position. Results are the CPU path's
 * bits (Stage.Forward, internal/llm/model.go:522-613). */
typedef struct rk_stage rk_stage;
typedef struct rk_moe rk_moe; /* a mixture-of-experts feed-forward (rk_moe_new, below) */

typedef struct {
    int32_t dim, hidden, heads, kv_heads;
    int32_t head_dim;   /* 0: dim/heads (internal/llm/model.go:66-71) */
    int32_t ctx;        /* positions the caches hold */
    int32_t qkv_bias;   /* Qwen2: q, k, v biases */
    int32_t qk_norm;    /* Qwen3: per-head RMSNorm of q and k before RoPE */
    float norm_eps;     /* Config.eps() (model.go:80-85) */
    float recip_dim;    /* num.Recip32(float32(dim)) (gpustage.go:124) */
    float recip_head;   /* num.Recip32(float32(head size)) (gpustage.go:125) */
    float inv_sqrt;     /* float32(1/math.Sqrt(float64(head size))) (gpustage.go:126) */
    int32_t seqs;       /* independent sequences decoded together (rk_stage_seqs_*); 0 or 1: one */
} rk_stage_config;

/* One layer: its uploaded Q8/Q4 matrices (internal/llm/model.go:150-166
 * Layer) and host copies of its vectors (NULL when the config has none).
 * With moe set, the layer's feed-forward is that mixture of experts (the
 * same RMSNorm before it and residual after it: x = Canonical(x + moe(xn)))
 * and w1, w2, w3 are not used (they may be NULL). */
typedef struct {
    rk_matrix *wq, *wk, *wv, *wo, *w1, *w2, *w3;
    const float *rms_att, *rms_ffn; /* dim */
    const float *bq, *bk, *bv;      /* q_dim, kv_dim, kv_dim (qkv_bias) */
    const float *q_norm, *k_norm;   /* head size (qk_norm) */
    rk_moe *moe;
} rk_stage_layer;

/* internal/llm/gpustage.go:51-83 newGPUStage: caches for ctx positions and
 * the rotary table rope_cos/rope_sin ([ctx][head size/2], NewRope,
 * internal/llm/model.go:428-441). Matrices stay owned by the caller and
 * must outlive the stage. */
int rk_stage_new(rk_device *dev, const rk_stage_config *c, const rk_stage_layer *layers, int32_t n_layers,
                 const float *rope_cos, const float *rope_sin, rk_stage **out);
/* internal/llm/gpustage.go:100-116 forward (Stage.ForwardMany): tokens
 * activations of dim floats at positions pos.., through the layers, in
 * place. Blocking. */
int rk_stage_forward(rk_stage *s, float *xs, int32_t pos, int32_t tokens);
/* Device bytes the stage holds beyond its matrices (internal/llm/
 * gpustage.go:90-98 ArenaBytes). */
int64_t rk_stage_bytes(const rk_stage *s);
/* internal/llm/gpustage.go:85-90 close. */
int rk_stage_free(rk_stage *s);

/* The coordinator's ends of a generation on the stage's device: the
 * embedding table (internal/llm/model.go:660-664 Embed), the head's final
 * RMSNorm and classifier (:667-673 Logits) and greedy sampling
 * (sample.go:45-53 argmax). embed and wcls may be the same matrix (a
 * shared classifier); rms_final is dim floats, copied. A stage with a head
 * holds every layer of the model. */
int rk_stage_set_head(rk_stage *s, rk_matrix *embed, rk_matrix *wcls, const float *rms_final);
/* Starts a greedy generation: the prompt's tokens at positions 0..n-1. */
int rk_stage_generate_start(rk_stage *s, const int32_t *prompt, int32_t n_prompt);
/* Runs the next `positions` positions (embed, layers, and at the prompt's
 * last position and after it the logits and the argmax, which becomes the
 * next position's token). logits, if not NULL, receives each run
 * position's vocab logits (positions before the prompt's last are left
 * as they were). Blocking. */
int rk_stage_generate_run(rk_stage *s, int32_t positions, float *logits);
/* Tokens at positions from..from+n-1 (prompt and generated). */
int rk_stage_generate_tokens(rk_stage *s, int32_t from, int32_t n, int32_t *out);
/* start, then run n_prompt+steps-1 positions: steps generated tokens. */
int rk_stage_generate(rk_stage *s, const int32_t *prompt, int32_t n_prompt, int32_t steps, int32_t *out);

/* Independent sequences decoded together (config.seqs of them; the
 * coordinator's generations, internal/llm/generate.go:415-522, run side by
 * side on one device). No reference counterpart as an API: each sequence's
 * tokens and logits are bit for bit those of its own generation alone
 * (rk_stage_generate), whatever the others hold. A stage of several
 * sequences runs only these (the single-sequence calls return RK_ERR_ARGS);
 * a stage of one runs both. The stage needs a head.
 *
 * start: prompts are the sequences' prompts back to back, lens[z] tokens
 * each (1..ctx); every prompt position but the last goes through the
 * batched path (each sequence's own caches). */
int rk_stage_seqs_start(rk_stage *s, const int32_t *prompts, const int32_t *lens);
/* `steps` decode steps: each sequence at its position (first the last of
 * its prompt) runs embed, layers and head; its greedy argmax becomes its
 * next token. logits, if not NULL, receives [steps][seqs][vocab]. Every
 * sequence's positions must stay within the context. Blocking; each step is
 * one replay of a recorded graph. */
int rk_stage_seqs_run(rk_stage *s, int32_t steps, float *logits);
/* Tokens of sequence `seq` at positions from..from+n-1. */
int rk_stage_seqs_tokens(rk_stage *s, int32_t seq, int32_t from, int32_t n, int32_t *out);
/* The next-token choice of sequence `seq` (0 on a stage of one sequence):
 * temperature <= 0 the greedy argmax (the default); otherwise a draw from
 * softmax(logits / temperature) with the xorshift64* generator seeded by
 * `seed` (0: the reference's fixed seed), bit for bit as the reference's
 * Sampler (internal/llm/sample.go:11-43; NewSampler per request at
 * internal/llm/generate.go:446, Sample per generated token at :538). The
 * state lives on the device, advances once per sampled token inside the
 * recorded step, and persists until set again: call it before each
 * generation for the reference's one sampler per request. */
int rk_stage_sampler(rk_stage *s, int32_t seq, float temperature, uint64_t seed);
/* The experts selected by the stage's MoE layers when several tokens run
 * together (independent sequences, prompt batches): the sum of each
 * grouping's distinct experts, and the number of groupings (one a MoE layer
 * a batch), since the stage was made or last asked; the counters restart.
 * No counterpart in the reference (which has no MoE model of this family):
 * it measures how much expert weight a batched step reads. */
int rk_stage_moe_stats(rk_stage *s, int64_t *selected, int64_t *groupings);
/* Sampler.Sample (internal/llm/sample.go:26-43) of `rows` rows of host
 * logits [rows][vocab] on the device: row z with temperature[z] and the
 * generator state state[z] (as NewSampler leaves it: a zero seed already
 * replaced), which advances when the row is sampled (temperature > 0 or
 * NaN); tokens[z] the pick. Blocking. */
int rk_sample_logits(rk_device *d, const float *logits, int64_t vocab, int32_t rows, const float *temperature,
                     uint64_t *state, int32_t *tokens);

/* ---- The device's float functions (internal/num), for host callers and
 * tests: out[i] = f(in[i]) computed by the same device code the kernels use.
 * No reference counterpart (the Go CPU path calls package num directly). */
enum { RK_FN_RECIP32 = 0, RK_FN_RSQRT32 = 1, RK_FN_EXP32 = 2, RK_FN_SILU = 3 };
int rk_num_eval(rk_device *dev, int32_t fn, const float *in, float *out, int64_t n);

/* ---- Mixture-of-experts feed-forward (config 5, Qwen3-MoE shape) ----
 * No counterpart in the reference's llama path: the contract is this
 * build's, after the order of internal/llm/dsv41/ops.go:67-74 (topK) and
 * forward.go:355-413 (moe). For each token's RMS-normed input xn:
 * z = router·xn (a Q8 product), p = softmax(z) (Go max, Exp32, one
 * sequential sum, Recip32; internal/llm/model.go:640-654), the top-k experts
 * by p (a stable order by cmp.Compare: larger first, lower index on ties,
 * NaN last), w_i = p_i·Recip32(Σ p_i) (the sum in selection order), and
 * y = Σ W2_e·(w_e·(silu(W1_e·xn)·(W3_e·xn))) over the selected experts in
 * ascending index, from +0, in float32. Experts are Q8 W1/W3 [hidden][dim]
 * and W2 [dim][hidden]; the router is Q8 [experts][dim]. The matrices stay
 * the caller's (free them after rk_moe_free, and after any stage that holds
 * the handle in a layer). */
int rk_moe_new(rk_device *dev, rk_matrix *router, int32_t experts, rk_matrix *const *w1, rk_matrix *const *w2,
               rk_matrix *const *w3, int32_t topk, rk_moe **out);
/* xn, y: [tokens][dim] host buffers; sel, wsel (either may be NULL):
 * [tokens][topk] selected experts and their weights. Blocking. */
int rk_moe_ffn(rk_moe *moe, const float *xn, int32_t tokens, float *y, int32_t *sel, float *wsel);
/* The same on device buffers, enqueued on `stream` (NULL: the device's). */
int rk_moe_ffn_device(rk_moe *moe, const float *d_xn, int32_t tokens, float *d_y, void *stream);
/* Device bytes of the scratch the handle keeps (grown to the largest batch). */
int64_t rk_moe_bytes(const rk_moe *moe);
int rk_moe_free(rk_moe *moe);

/* ---- rakkan_tensor_v1 operators (internal/sandbox/tensor.go) ----
 * Element types as the tensor table's (tensor.go:42-44). */
enum { RK_TENSOR_F32 = 0, RK_TENSOR_I8 = 1, RK_TENSOR_I32 = 2 };

/* tensor.go:286-339 tenMatmul: c = a[m,k]·b with b[k,n] (transposed = 0,
 * matmul) or b[n,k] (transposed = 1, matmul_t). RK_TENSOR_F32: f32 in and
 * out, acc += float32(a·b) for p = 0..k-1 from +0, Canonical(acc).
 * RK_TENSOR_I8: int8 in, int32 out, Go int32 wraparound. Any other dtype
 * (i32 inputs included) or a dimension outside 1..2^24 (tensor.go:60) is
 * RK_ERR_ARGS, as tenErrArgs (-1). The caller charges gas m·n·k·8 and keeps
 * the memory budget (tensor.go:300-310) before calling. Host buffers,
 * blocking. */
int rk_tensor_matmul(rk_device *dev, int32_t dtype, int32_t transposed, int64_t m, int64_t k, int64_t n,
                     const void *a, const void *b, void *c);
/* The same on device-resident a, b, c, enqueued on `stream` (NULL: the
 * device's own) without waiting. */
int rk_tensor_matmul_device(rk_device *dev, int32_t dtype, int32_t transposed, int64_t m, int64_t k, int64_t n,
                            const void *d_a, const void *d_b, void *d_c, void *stream);
/* tensor.go:445-461 tenQuantize: q = int8(max(-127, min(127,
 * float32(RoundToEven(v/k))))) with a true f32 division; k > 0. A NaN
 * quotient gives 0 (amd64's conversion of NaN). */
int rk_tensor_quantize(rk_device *dev, const float *a, int8_t *q, int64_t n, float k);
/* tensor.go:366-387 tenScale: out = Canonical(float32(v)·k) for an f32 or
 * i32 input (dtype RK_TENSOR_F32 / RK_TENSOR_I32; i8 is RK_ERR_ARGS). */
int rk_tensor_scale(rk_device *dev, int32_t dtype, const void *a, float *out, int64_t n, float k);

/* The tensor ABI across the worker process. The reference runs the tensor
 * operators in an isolated worker whose seccomp allow-list has read and
 * write on inherited descriptors but no ioctl or openat
 * (internal/isolate/seccomp_linux_amd64.go:10-38): the worker cannot open a
 * GPU. So the node process, which owns the device, serves the worker's
 * products over a descriptor the worker inherits
 * (internal/isolate/inherit_unix.go:10). The worker keeps tenMatmul's
 * checks and gas (internal/sandbox/tensor.go:286-339) and sends the operands;
 * the node answers with rk_tensor_matmul's result. Wire format (little-
 * endian): a request is a 56-byte header {u32 'RKTQ', u32 op = 1 (matmul),
 * i32 dtype, i32 transposed, i64 m, k, n, u64 a_bytes, b_bytes} then a's and
 * b's bytes; a reply is {u32 'RKTA', i32 status, u64 c_bytes} then, for
 * status 0, c's bytes. No reference counterpart as code: the reference's
 * tensor operators run on the worker's CPU.
 *
 * Node side: serves requests from fd until the worker closes its end
 * (returns RK_OK), each answered with rk_tensor_matmul's status and result
 * (a device error is answered and serving goes on). A malformed request
 * (magic, op, dtype, a dimension outside 1..2^24, sizes that do not match
 * the dimensions) is answered with RK_ERR_ARGS and ends serving with
 * RK_ERR_ARGS; one whose a + b + c bytes pass max_bytes (0: 1 GiB) with
 * RK_ERR_OOM; a broken stream returns RK_ERR_HIP. Blocking; one call serves
 * one worker, so several workers take one thread each. */
int rk_tensor_serve(rk_device *dev, int32_t fd, int64_t max_bytes);
/* The worker side, rk_tensor_call, is in librkworker.so (rk_worker.h): a
 * host-only library, so the worker loads none of the GPU runtime. */

/* internal/gpu/profile.go:82-109 StartProfile / StopProfile. While a
 * profile is active, every kernel the library launches is bracketed by HIP
 * events on the stream it runs on; stop waits for them and returns, per
 * kernel, the launches and their summed duration, the slowest first (at most
 * cap entries written, *n = entries available). */
typedef struct {
    char kernel[48];
    int64_t calls;
    double ms;
} rk_profile_entry;

int rk_profile_start(rk_device *dev);
int rk_profile_stop(rk_device *dev, rk_profile_entry *out, int32_t cap, int32_t *n);

/* ---- Diagnostics (no counterpart in the reference) ----
 * The floor under one launch on this device, for reading a product's time
 * against: the time per launch of `launches` back-to-back launches of an
 * empty kernel (*empty_us) and of a plain streaming read of `bytes` (a
 * multiple of 16) that stores nothing (*read_us). The reads take `copies`
 * buffers in turn, so that copies·bytes past the 256 MB MALL come from HBM.
 * Allocates copies·bytes of device memory for the call. */
int rk_device_launch_floor(rk_device *dev, int64_t bytes, int32_t copies, int32_t launches, float *empty_us,
                           float *read_us);

#ifdef __cplusplus
}
#endif
#endif
