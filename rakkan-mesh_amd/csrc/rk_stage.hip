// rk_stage.hip — stages: llama-family layers resident on one device
// (internal/llm/gpustage.go), and the greedy generation loop around them
// (embedding, head, argmax) with its state on the device.
//
// A token runs as six launches per layer; each product takes its input
// quantized, or normalizes and quantizes it in its own prologue:
//   qkv      xn = RMSNorm_att(x) (prologue; layer 0: the embedding kernel's),
//            [Wq;Wk;Wv]·xn (+bias), RoPE, k and v into the caches
//            (Qwen3: raw q/k/v, then qknorm_rope)
//   scores   Dot32(q_h, k_t)·invSqrt for t <= position
//   values   softmax, Σ a_t·v_t, quantized
//   wo       x += Wo·att
//   w13      xn = RMSNorm_ffn(x) (prologue), h = silu(W1·xn)·(W3·xn), quantized
//   w2       x = Canonical(x + W2·h)
// and the head's norm runs in the classifier's prologue.
// in the order and rounding of Stage.Forward (internal/llm/model.go:522-613).
// Generation embeds the position's token first (and RMSNorms it for the
// first layer) and ends with the classifier and the greedy argmax, which
// writes the next token and advances the position on the device. The
// launches of one token are recorded once into a HIP graph and replayed.
#include <cstring>
#include <vector>

#include "rk_fused.h"
#include "rk_layer.h"
#include "rk_mm.h"
#include "rk_moe.h"
#include "rk_runtime.h"

// internal/llm/gpustage.go:23-32 gpuStage.
struct rk_stage {
    rk_device *d = nullptr;
    rk_stage_config c{};
    int hs = 0, qdim = 0, kvdim = 0, half = 0;
    std::vector<rk_stage_layer> layers;
    char *mem = nullptr;  // one device allocation for all of the below
    int64_t bytes = 0;
    float *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *att_out = nullptr;
    float *h = nullptr, *cos_t = nullptr, *sin_t = nullptr, *logits = nullptr, *rms_final = nullptr;
    int64_t logits_n = 0;  // floats of logits (and of its pinned staging)
    int64_t logits_dev = 0;  // floats of the logits allocation (logits, then the sampler's terms)
    // The next-token choice (rk_stage_sampler): temperatures and xorshift64*
    // states per sequence on the device, the sampler's scratch (terms after
    // the logits), and whether any sequence samples (the recorded step then
    // ends with the sampler instead of the greedy argmax).
    float *smp_temp = nullptr, *smp_part = nullptr, *smp_terms = nullptr;
    uint64_t *smp_state = nullptr;
    std::vector<float> smp_t;
    bool sampling = false;
    int32_t *ctl = nullptr, *tokens = nullptr;
    unsigned long long *amax = nullptr;  // the classifier's argmax keys
    int8_t *qx = nullptr;  // the fallback quantize's output
    float *xs = nullptr;
    int32_t *xsum = nullptr;
    // Quantized inputs passed between launches: A (attention -> Wo, W1/W3
    // -> W2) and B (norm tails and the embedding -> QKV, W1/W3, classifier).
    rk::QScratch qa{}, qb{};
    struct LayerDev {
        float *rms_att, *rms_ffn, *bias, *q_norm, *k_norm;  // device copies
        float *keys, *vals;
    };
    std::vector<LayerDev> ld;
    // head (rk_stage_set_head)
    rk_matrix *embed = nullptr, *wcls = nullptr;
    // pinned staging of rk_stage_forward / generate
    float *h_x = nullptr;
    int32_t *h_ctl = nullptr;
    float *h_logits = nullptr;
    // recorded tokens: layers only (forward), or the whole generation step
    hipGraph_t g_layers = nullptr, g_token = nullptr;
    hipGraphExec_t x_layers = nullptr, x_token = nullptr;
    // Batches of consecutive positions (a forward of several tokens): rows
    // [bcap][...] of the residual, q/k/v, scores, attention output and the
    // two quantized inputs; one allocation, made on first use.
    int bcap = 0;
    int32_t prompt_n = 0;  // the current generation's prompt length
    char *bmem = nullptr;
    int64_t bbytes = 0;
    float *bx = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr, *batt = nullptr, *batt_out = nullptr;
    rk::QScratch bqa{}, bqb{};
    // Independent sequences (rk_stage_seqs_*): each has its own caches
    // (sequence z's at z·ctx·kv_dim in every layer's), position, prompt
    // length and tokens [ctx+1] on the device; the host keeps a copy of the
    // positions for the context bound.
    int seqs = 1;
    int32_t *seq_pos = nullptr, *seq_prompt = nullptr, *seq_tokens = nullptr;
    int32_t *h_seq = nullptr;
    std::vector<int32_t> seq_at;
    bool seqs_started = false;
    hipGraph_t g_seqs = nullptr;
    hipGraphExec_t x_seqs = nullptr;
    // Mixture-of-experts layers share one scratch (they run one after
    // another), laid out per layer for moe_cap tokens.
    char *moe_mem = nullptr;
    int moe_cap = 0;
    // the groupings' counters (MoeScratch::stat): experts selected, groupings
    unsigned long long *moe_stat = nullptr;
    // the hand-off words of the values-and-Wo launch (kSyncWords; its
    // kSyncError is also the MoE launches' error word)
    unsigned long long *sync = nullptr;
    // each MoE layer's hand-off words for its one-token launch (a stride
    // of moe_sync_stride words)
    unsigned long long *moe_sync = nullptr;
    int64_t moe_sync_stride = 0;
};

namespace rk {

static constexpr int kForwardBatch = 64;  // tokens per staging round (gpustage.go:17)

static int fmt_of(const rk_matrix *m) { return m->kind == RK_Q4 ? kFmtQ4 : kFmtQ8; }

// One product of a stage: matrices ms[0..n) of one format, epilogue epi;
// input quantized in q, or (q null) f32 `in` quantized by the product's own
// prologue, RMSNorm'd with `norm` first when given (or, too wide for that,
// by a separate launch into s->qx).
static int stage_product(rk_stage *s, hipStream_t st, const char *name, const QScratch *q, const float *in,
                         const float *norm, rk_matrix *const *ms, int n, float *const *outs, int epi, FusedArgs a) {
    rk_device *d = s->d;
    const int cols = (int)ms[0]->cols;
    const int fmt = fmt_of(ms[0]);
    a.nseg = n;
    a.cols = cols;
    int64_t rows = 0;
    for (int i = 0; i < n; i++) {
        a.seg[i] = MatSeg{ms[i]->w, ms[i]->scales, outs ? outs[i] : nullptr, ms[i]->rows};
        rows += ms[i]->rows;
    }
    a.rows = (int32_t)rows;
    int pro = kProGlobal;
    if (q) {
        a.qx = q->qx;
        a.xs = q->xs;
        a.xsum = q->xsum;
    } else if (norm && fused_fits(kProNorm, cols)) {
        pro = kProNorm;
        a.x = in;
        a.norm_w = norm;
        a.recip_n = s->c.recip_dim;
        a.norm_eps = s->c.norm_eps;
    } else if (!norm && fused_fits(kProQuant, cols)) {
        pro = kProQuant;
        a.x = in;
    } else {
        if (norm) {
            ProfScope p(d, st, "norm_quant");
            launch_norm_quant(in, cols, norm, s->c.recip_dim, s->c.norm_eps, s->qx, s->xs, s->xsum, st);
        } else {
            ProfScope p(d, st, "quantize_acts");
            launch_quantize_acts(in, cols, s->qx, s->xs, s->xsum, st);
        }
        a.qx = s->qx;
        a.xs = s->xs;
        a.xsum = s->xsum;
    }
    bool ok;
    {
        ProfScope p(d, st, name);
        ok = launch_fused(fmt, pro, epi, a, d->cu, st);
    }
    if (!ok) return fail(d, RK_ERR_UNSUPPORTED, "stage: %s product of width %d has no kernel", name, cols);
    return RK_OK;
}

// The attention of the position in ctl (or of a batch, bt): the scores
// into att, then the softmax and the weighted values (quantized into qo
// when given). Two launches: the scores need many workgroups (every score
// reads a whole key row), the sequential sums few. (One launch computing
// a head's scores in the workgroups of its value sums measured slower on
// MI355X: each workgroup then reads all of the head's keys.)
// The raw k and v rows and the norm weights of a QK-norm layer: attention
// then starts with the norm and RoPE of q and k and the caches' store.
struct QkNorm {
    const float *k, *v, *q_norm, *k_norm;
};

// wo (a decode step, qo given): the attention output's Wo product added
// into the residual x in the values launch when launch_att_values_wo takes
// the shapes; the return says whether it did.
static bool enqueue_attention(rk_stage *s, hipStream_t st, const float *q, float *keys, float *vals, float *att,
                              float *out, const int32_t *ctl, const AttBatch &bt, const QScratch *qo,
                              const QkNorm *qk = nullptr, const rk_matrix *wo = nullptr, float *x = nullptr) {
    rk_device *d = s->d;
    const rk_stage_config &c = s->c;
    int8_t *qx = qo ? qo->qx : nullptr;
    float *xs = qo ? qo->xs : nullptr;
    int32_t *xsum = qo ? qo->xsum : nullptr;
    bool scored = false;
    if (qk && wo && wo->kind == RK_Q8 && ctl && qo) {
        // a decode step of a QK-norm layer: the scores formed in the values
        // launch (contexts up to 256)
        const QknIn in{q,    qk->k, qk->v,        qk->q_norm, qk->k_norm, s->cos_t, s->sin_t,
                       keys, vals,  c.recip_head, c.norm_eps, c.inv_sqrt};
        ProfScope p(d, st, "att_values_wo");
        if (launch_att_values_wo(att, c.ctx, vals, out, ctl, c.ctx, c.heads, c.kv_heads, s->hs, s->kvdim, qx, xs, xsum,
                                 wo->w, wo->scales, wo->rows, wo->cols, x, s->sync, st, &in))
            return true;
    }
    if (qk) {
        {
            // a decode step or independent sequences: the norm folded into
            // the scores launch
            ProfScope p(d, st, "att_scores");
            scored = launch_att_scores_qkn(q, qk->k, qk->v, qk->q_norm, qk->k_norm, c.recip_head, c.norm_eps,
                                           s->cos_t, s->sin_t, keys, vals, att, c.ctx, ctl, bt, c.ctx, c.heads,
                                           c.kv_heads, s->hs, s->kvdim, c.inv_sqrt, st);
        }
        if (!scored) {
            ProfScope p(d, st, "qknorm_rope");
            launch_qknorm_rope(const_cast<float *>(q), qk->k, qk->v, qk->q_norm, qk->k_norm, c.recip_head, c.norm_eps,
                               s->cos_t, s->sin_t, ctl, bt.pos0, bt.tokens, keys, vals, c.heads, c.kv_heads, s->hs, st,
                               bt.pos, bt.cache_stride);
        }
    }
    if (!scored) {
        ProfScope p(d, st, "att_scores");
        launch_att_scores(q, keys, att, c.ctx, ctl, bt, c.ctx, c.heads, c.kv_heads, s->hs, s->kvdim, c.inv_sqrt, st);
    }
    if (wo && wo->kind == RK_Q8 && ctl && qo) {
        ProfScope p(d, st, "att_values_wo");
        if (launch_att_values_wo(att, c.ctx, vals, out, ctl, c.ctx, c.heads, c.kv_heads, s->hs, s->kvdim, qx, xs, xsum,
                                 wo->w, wo->scales, wo->rows, wo->cols, x, s->sync, st))
            return true;
    }
    ProfScope p(d, st, "att_values");
    launch_att_values(att, c.ctx, vals, out, ctl, bt, c.ctx, c.heads, c.kv_heads, s->hs, s->kvdim, qx, xs, xsum, st,
                      d->cu);
    return false;
}

// The launches of one layer (Stage.Forward's body, model.go:530-611). The
// norms run in the prologues of the products that read them (QKV: the
// attention norm, unless qb already holds it; W1/W3: the ffn norm).
static int enqueue_layer(rk_stage *s, int li, hipStream_t st, bool qb_ready) {
    rk_device *d = s->d;
    const rk_stage_config &c = s->c;
    const rk_stage_layer &L = s->layers[li];
    const rk_stage::LayerDev &D = s->ld[li];
    int rc;
    FusedArgs base{};
    base.ctl = s->ctl;
    base.hs = s->hs;
    base.qdim = s->qdim;
    base.kvdim = s->kvdim;
    // q, k, v: runs of consecutive matrices of one format share a launch.
    rk_matrix *qkv[3] = {L.wq, L.wk, L.wv};
    if (!c.qk_norm) {
        base.cos_t = s->cos_t;
        base.sin_t = s->sin_t;
        base.kcache = D.keys;
        base.vcache = D.vals;
        base.bias = D.bias;
        int i = 0, row = 0;
        while (i < 3) {
            int j = i + 1;
            while (j < 3 && qkv[j]->kind == qkv[i]->kind) j++;
            FusedArgs a = base;
            a.row_base = row;  // the epilogue indexes q/k/v rows and biases by row_base + row
            float *outs[3] = {i == 0 ? s->q : nullptr, nullptr, nullptr};  // only q rows store through seg[0]
            if ((rc = stage_product(s, st, "qkv", qb_ready ? &s->qb : nullptr, s->x, qb_ready ? nullptr : D.rms_att,
                                    qkv + i, j - i, outs, kEpQKV, a)))
                return rc;
            for (int t = i; t < j; t++) row += (int)qkv[t]->rows;
            i = j;
        }
    } else {
        float *outs[3] = {s->q, s->k, s->v};
        int i = 0;
        while (i < 3) {
            int j = i + 1;
            while (j < 3 && qkv[j]->kind == qkv[i]->kind) j++;
            FusedArgs a = base;
            int row = 0;
            for (int t = 0; t < i; t++) row += (int)qkv[t]->rows;
            a.bias = D.bias ? D.bias + row : nullptr;
            if ((rc = stage_product(s, st, "qkv", qb_ready ? &s->qb : nullptr, s->x, qb_ready ? nullptr : D.rms_att,
                                    qkv + i, j - i, outs + i, kEpStore, a)))
                return rc;
            i = j;
        }
    }
    // The attention output comes quantized when its Q8 blocks fall within
    // heads (head size a multiple of 32).
    const bool att_q = s->hs % 32 == 0;
    const QkNorm qk{s->k, s->v, D.q_norm, D.k_norm};
    const bool wo_done = enqueue_attention(s, st, s->q, D.keys, D.vals, s->att, s->att_out, s->ctl, AttBatch{},
                                           att_q ? &s->qa : nullptr, c.qk_norm ? &qk : nullptr, L.wo, s->x);
    float *xo[1] = {s->x};
    if (!wo_done &&
        (rc = stage_product(s, st, "wo", att_q ? &s->qa : nullptr, s->att_out, nullptr, &L.wo, 1, xo, kEpAdd, base)))
        return rc;
    if (L.moe) {
        // a mixture of experts: its input RMSNorm_ffn(x) quantized into qb;
        // the experts' sum goes into the residual, x = Canonical(x + y)
        MoeScratch sc;
        moe_scratch_layout(L.moe, s->moe_cap, s->moe_mem, &sc);
        sc.stat = s->moe_stat;
        sc.sync = s->moe_sync + (int64_t)li * s->moe_sync_stride;
        sc.err = s->sync + kSyncError;
        return enqueue_moe_x(L.moe, sc, s->x, D.rms_ffn, c.recip_dim, c.norm_eps, 1, s->qb.qx, s->qb.xs, s->qb.xsum,
                             s->x, true, st);
    }
    // W1 row r and W3 row r interleaved (logical rows); h leaves quantized in qa.
    rk_matrix *w13[2] = {L.w1, L.w3};
    float *ho[2] = {s->h, nullptr};
    FusedArgs a13 = base;
    a13.qx_out = s->qa.qx;
    a13.xs_out = s->qa.xs;
    a13.xsum_out = s->qa.xsum;
    if ((rc = stage_product(s, st, "w13", nullptr, s->x, D.rms_ffn, w13, 2, ho, kEpSilu, a13))) return rc;
    if ((rc = stage_product(s, st, "w2", &s->qa, nullptr, nullptr, &L.w2, 1, xo, kEpAddCanon, base))) return rc;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(d, e, "stage launch");
    return RK_OK;
}

// All layers on x; qb_ready: qb already holds the first layer's normed
// input (the embedding kernel's).
static int enqueue_layers(rk_stage *s, hipStream_t st, bool qb_ready) {
    const int n = (int)s->layers.size();
    for (int li = 0; li < n; li++) {
        int rc = enqueue_layer(s, li, st, li == 0 && qb_ready);
        if (rc) return rc;
    }
    return RK_OK;
}

// Layers on the activation the host wrote to x.
static int enqueue_forward(rk_stage *s, hipStream_t st) { return enqueue_layers(s, st, false); }

// The sampler's launch for `seqs` logits rows (SampleArgs).
static SampleArgs sample_args(rk_stage *s, int seqs, int32_t *pos, const int32_t *prompt, int32_t *tokens,
                              int64_t tok_stride, unsigned long long *amax) {
    SampleArgs a{};
    a.logits = s->logits;
    a.vocab = s->wcls->rows;
    a.seqs = seqs;
    a.pos = pos;
    a.prompt = prompt;
    a.tokens = tokens;
    a.tok_stride = tok_stride;
    a.tokens_len = s->c.ctx + 1;
    a.temps = s->smp_temp;
    a.states = s->smp_state;
    a.terms = s->smp_terms;
    a.part = s->smp_part;
    a.amax = amax;
    return a;
}

// One generation step: embed the position's token, the layers, the head.
static int enqueue_token(rk_stage *s, hipStream_t st) {
    rk_device *d = s->d;
    {
        ProfScope p(d, st, "embed");
        launch_embed_norm(s->embed->w, s->embed->scales, s->embed->kind == RK_Q4, s->tokens, s->ctl, s->c.dim, s->x,
                          s->ld[0].rms_att, s->c.recip_dim, s->c.norm_eps, s->qb.qx, s->qb.xs, s->qb.xsum, st);
    }
    int rc = enqueue_layers(s, st, true);
    if (rc) return rc;
    FusedArgs a{};
    a.ctl = s->ctl;
    a.amax = s->amax;
    a.gate = 1;
    float *lo[1] = {s->logits};
    if ((rc = stage_product(s, st, "logits", nullptr, s->x, s->rms_final, &s->wcls, 1, lo, kEpLogits, a))) return rc;
    if (s->sampling) {
        ProfScope p(d, st, "sample");
        launch_sample(sample_args(s, 1, s->ctl + kCtlPos, s->ctl + kCtlPrompt, s->tokens, 0, s->amax), st);
    } else {
        ProfScope p(d, st, "advance");
        launch_advance(s->ctl, s->amax, s->tokens, s->c.ctx + 1, st);
    }
    return RK_OK;
}

// What a stage records: its layers (Stage.ForwardMany), a whole generation
// step, or a decode step of every sequence.
enum Rec { kRecLayers, kRecToken, kRecSeqs };

static int enqueue_rec(rk_stage *s, Rec which, hipStream_t st);

// Records `which` into a graph, once.
static int record(rk_stage *s, Rec which) {
    rk_device *d = s->d;
    hipGraph_t &g = which == kRecToken ? s->g_token : which == kRecSeqs ? s->g_seqs : s->g_layers;
    hipGraphExec_t &x = which == kRecToken ? s->x_token : which == kRecSeqs ? s->x_seqs : s->x_layers;
    if (x) return RK_OK;
    HIP_TRY(d, hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal), "stage capture");
    d->capturing = true;
    int rc = enqueue_rec(s, which, d->stream);
    d->capturing = false;
    hipGraph_t gr = nullptr;
    hipError_t e = hipStreamEndCapture(d->stream, &gr);
    if (rc) {
        if (gr) (void)hipGraphDestroy(gr);
        return rc;
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return hip_fail(d, e, "stage capture");
    }
    e = hipGraphInstantiate(&x, gr, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(gr);
        (void)hipGetLastError();
        x = nullptr;
        return hip_fail(d, e, "stage graph");
    }
    g = gr;
    return RK_OK;
}

// After the stream is idle: whether a launch with an in-launch hand-off
// (values and Wo, a one-token MoE feed-forward) gave up waiting for its
// input (kSyncError; its results are then not the product).
static int sync_check(rk_stage *s, const char *what) {
    rk_device *d = s->d;
    unsigned long long err = 0;
    HIP_TRY(d, hipMemcpy(&err, s->sync + kSyncError, sizeof err, hipMemcpyDeviceToHost), what);
    if (err) return fail(d, RK_ERR_HIP, "%s: a launch timed out waiting for a hand-off inside it", what);
    return RK_OK;
}

// Runs the recorded `which` once on the device stream; while the device
// profiles, the launches run one by one instead, each timed.
static int run_once(rk_stage *s, Rec which) {
    rk_device *d = s->d;
    if (d->profiling) return enqueue_rec(s, which, d->stream);
    int rc = record(s, which);
    if (rc) return rc;
    HIP_TRY(d, hipGraphLaunch(which == kRecToken ? s->x_token : which == kRecSeqs ? s->x_seqs : s->x_layers, d->stream),
            "stage replay");
    return RK_OK;
}

// ---- Batches of consecutive positions (prompt prefill) ----
// The same per-token operations as enqueue_layer, each launch covering n
// tokens at positions pos0..pos0+n-1: products on int8 MFMA (rk_mm.hip),
// norms one workgroup per token, attention one grid slice per token. Every
// token's results are those of its own decode-path forward, bit for bit.

// Largest batch the buffers take: 256 tokens, fewer when the scores of a
// batch ([tokens][heads][ctx] floats) would pass 512 MiB, and never fewer
// than the stage's sequences (one row each in a decode step).
static int batch_cap(const rk_stage_config &c, int seqs) {
    const int64_t per = (int64_t)4 * c.heads * c.ctx;
    int64_t cap = ((int64_t)512 << 20) / std::max<int64_t>(per, 1);
    cap = std::min<int64_t>(cap, 256);
    return (int)std::max<int64_t>(std::max<int64_t>(cap, 1), seqs);
}

// Where a batch's tokens sit: consecutive positions pos0, pos0+1, ... of
// one sequence whose caches start cache0 floats into each layer's (a
// prompt), or one token per sequence, token z at seq_pos[z] in caches
// cache_stride floats apart (the sequences' decode step).
struct BatchPos {
    int32_t pos0 = 0;
    const int32_t *seq_pos = nullptr;
    int64_t cache0 = 0, cache_stride = 0;
};

static int batch_alloc(rk_stage *s) {
    if (s->bmem) return RK_OK;
    rk_device *d = s->d;
    const rk_stage_config &c = s->c;
    const int64_t B = batch_cap(c, s->seqs);
    const int64_t widest = std::max<int64_t>(std::max<int64_t>(c.dim, s->qdim), c.hidden);
    std::vector<std::pair<void **, int64_t>> plan;
    auto take = [&](void **p, int64_t n) { plan.push_back({p, n}); };
    take((void **)&s->bx, 4 * B * c.dim);
    take((void **)&s->bq, 4 * B * s->qdim);
    take((void **)&s->bk, 4 * B * s->kvdim);
    take((void **)&s->bv, 4 * B * s->kvdim);
    take((void **)&s->batt, 4 * B * c.heads * c.ctx);
    take((void **)&s->batt_out, 4 * B * s->qdim);
    for (QScratch *q : {&s->bqa, &s->bqb}) {
        take((void **)&q->qx, B * widest);
        take((void **)&q->xs, 4 * B * (widest / 32));
        take((void **)&q->xsum, 4 * B * (widest / 32));
    }
    int64_t at = 0;
    for (auto &pl : plan) at += (pl.second + 255) & ~(int64_t)255;
    int rc = dev_alloc(d, (void **)&s->bmem, (size_t)at, "stage batch");
    if (rc) return rc;
    s->bbytes = at;
    at = 0;
    for (auto &pl : plan) {
        *pl.first = s->bmem + at;
        at += (pl.second + 255) & ~(int64_t)255;
    }
    s->bcap = (int)B;
    s->bytes += s->bbytes;
    add_used(d, s->bbytes);
    return RK_OK;
}

// One batched product: matrices ms[0..n) of one format (concatenated rows;
// kEpSilu: W1 and W3 paired).
static int batch_product(rk_stage *s, hipStream_t st, const char *name, rk_matrix *const *ms, int n, int epi,
                         MmArgs a) {
    rk_device *d = s->d;
    a.nseg = n;
    a.cols = (int32_t)ms[0]->cols;
    a.rows = 0;
    for (int i = 0; i < n; i++) {
        a.seg[i].w = ms[i]->w;
        a.seg[i].ws = ms[i]->scales;
        a.seg[i].rows = ms[i]->rows;
        if (epi != kEpSilu || i == 0) a.rows += (int32_t)ms[i]->rows;
    }
    bool ok;
    {
        ProfScope p(d, st, name);
        ok = launch_mm(fmt_of(ms[0]), epi, a, st);
    }
    if (!ok) return fail(d, RK_ERR_UNSUPPORTED, "stage: batched %s product has no kernel", name);
    return RK_OK;
}

// RMSNorm of the batch's rows with w, quantized into bqb.
static void batch_norm(rk_stage *s, hipStream_t st, const float *w, int n) {
    if (!w) return;
    ProfScope p(s->d, st, "norm_quant");
    launch_norm_quant(s->bx, s->c.dim, w, s->c.recip_dim, s->c.norm_eps, s->bqb.qx, s->bqb.xs, s->bqb.xsum, st, n);
}

// One layer for n tokens placed as bp says; on entry bqb holds their
// RMSNorm_att(x) quantized.
static int enqueue_layer_batch(rk_stage *s, int li, hipStream_t st, int n, const BatchPos &bp,
                               const float *next_norm) {
    rk_device *d = s->d;
    const rk_stage_config &c = s->c;
    const rk_stage_layer &L = s->layers[li];
    const rk_stage::LayerDev &D = s->ld[li];
    int rc;
    MmArgs base{};
    base.tokens = n;
    base.qx = s->bqb.qx;
    base.xs = s->bqb.xs;
    rk_matrix *qkv[3] = {L.wq, L.wk, L.wv};
    int i = 0, row = 0;
    while (i < 3) {  // runs of consecutive matrices of one format share a launch
        int j = i + 1;
        while (j < 3 && qkv[j]->kind == qkv[i]->kind) j++;
        MmArgs a = base;
        if (!c.qk_norm) {
            a.row_base = row;
            a.bias = D.bias;
            a.pos0 = bp.pos0;
            a.seq_pos = bp.seq_pos;
            a.cache_stride = bp.cache_stride;
            a.hs = s->hs;
            a.qdim = s->qdim;
            a.kvdim = s->kvdim;
            a.cos_t = s->cos_t;
            a.sin_t = s->sin_t;
            a.q = s->bq;
            a.kcache = D.keys + bp.cache0;
            a.vcache = D.vals + bp.cache0;
            if ((rc = batch_product(s, st, "qkv", qkv + i, j - i, kEpQKV, a))) return rc;
        } else {
            float *outs[3] = {s->bq, s->bk, s->bv};
            for (int t = i; t < j; t++) a.seg[t - i].out = outs[t];
            a.bias = D.bias ? D.bias + row : nullptr;
            if ((rc = batch_product(s, st, "qkv", qkv + i, j - i, kEpStore, a))) return rc;
        }
        for (int t = i; t < j; t++) row += (int)qkv[t]->rows;
        i = j;
    }
    AttBatch bt;
    bt.pos0 = bp.pos0;
    bt.tokens = n;
    bt.q_stride = s->qdim;
    bt.att_stride = (int64_t)c.heads * c.ctx;
    bt.out_stride = s->qdim;
    bt.pos = bp.seq_pos;
    bt.cache_stride = bp.cache_stride;
    // the attention output comes quantized when its Q8 blocks fall within
    // heads; else it is quantized by a launch of its own
    const bool att_q = s->hs % 32 == 0;
    const QkNorm qk{s->bk, s->bv, D.q_norm, D.k_norm};
    enqueue_attention(s, st, s->bq, D.keys + bp.cache0, D.vals + bp.cache0, s->batt, s->batt_out, nullptr, bt,
                      att_q ? &s->bqa : nullptr, c.qk_norm ? &qk : nullptr);
    if (!att_q) {
        ProfScope p(d, st, "quantize_acts");
        launch_quantize_acts(s->batt_out, (int64_t)n * s->qdim, s->bqa.qx, s->bqa.xs, s->bqa.xsum, st);
    }
    MmArgs a = base;
    a.qx = s->bqa.qx;
    a.xs = s->bqa.xs;
    a.x = s->bx;
    a.ldx = c.dim;
    if ((rc = batch_product(s, st, "wo", &L.wo, 1, kEpAdd, a))) return rc;
    if (L.moe) {  // RMSNorm_ffn(x) into bqb, and the experts' sums into the residual rows, x = Canonical(x + y)
        MoeScratch sc;
        moe_scratch_layout(L.moe, s->moe_cap, s->moe_mem, &sc);
        sc.stat = s->moe_stat;
        // the sum's launch also forms the next layer's normed input in bqb
        const MoeNext nx{next_norm, c.recip_dim, c.norm_eps, s->bqb.qx, s->bqb.xs, s->bqb.xsum};
        if ((rc = enqueue_moe_x(L.moe, sc, s->bx, D.rms_ffn, c.recip_dim, c.norm_eps, n, s->bqb.qx, s->bqb.xs,
                                s->bqb.xsum, s->bx, true, st, next_norm ? &nx : nullptr)))
            return rc;
        hipError_t e = hipGetLastError();
        return e == hipSuccess ? RK_OK : hip_fail(d, e, "stage launch");
    }
    batch_norm(s, st, D.rms_ffn, n);
    rk_matrix *w13[2] = {L.w1, L.w3};
    a = base;
    a.qx_out = s->bqa.qx;
    a.xs_out = s->bqa.xs;
    a.xsum_out = s->bqa.xsum;
    if ((rc = batch_product(s, st, "w13", w13, 2, kEpSilu, a))) return rc;
    a = base;
    a.qx = s->bqa.qx;
    a.xs = s->bqa.xs;
    a.x = s->bx;
    a.ldx = c.dim;
    if ((rc = batch_product(s, st, "w2", &L.w2, 1, kEpAddCanon, a))) return rc;
    batch_norm(s, st, next_norm, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(d, e, "stage launch");
    return RK_OK;
}

// Every layer over n tokens whose activations are in bx.
static int enqueue_forward_batch(rk_stage *s, hipStream_t st, int n, const BatchPos &bp) {
    batch_norm(s, st, s->ld[0].rms_att, n);
    const int nl = (int)s->layers.size();
    for (int li = 0; li < nl; li++) {
        int rc = enqueue_layer_batch(s, li, st, n, bp, li + 1 < nl ? s->ld[li + 1].rms_att : nullptr);
        if (rc) return rc;
    }
    return RK_OK;
}

static BatchPos at_pos(int32_t pos0) {
    BatchPos bp;
    bp.pos0 = pos0;
    return bp;
}

// One decode step of every sequence (rk_stage_seqs_run): sequence z's token
// at seq_pos[z] embedded into row z, the layers (each row attends to its
// own sequence's caches), the head's RMSNorm and classifier for every row,
// and the greedy step that writes each sequence's next token and advances
// its position. Every position is read on the device, so the step is
// recorded once and replayed.
static int enqueue_seqs_step(rk_stage *s, hipStream_t st) {
    rk_device *d = s->d;
    const rk_stage_config &c = s->c;
    const int S = s->seqs;
    const int64_t ctx = c.ctx;
    {
        ProfScope p(d, st, "embed");
        launch_embed_rows(s->embed->w, s->embed->scales, s->embed->kind == RK_Q4, s->seq_tokens, 0, S, c.dim, s->bx,
                          st, ctx + 1, s->seq_pos);
    }
    BatchPos bp;
    bp.seq_pos = s->seq_pos;
    bp.cache_stride = ctx * s->kvdim;
    int rc = enqueue_forward_batch(s, st, S, bp);
    if (rc) return rc;
    batch_norm(s, st, s->rms_final, S);
    MmArgs a{};
    a.seg[0] = MatSeg{s->wcls->w, s->wcls->scales, s->logits, s->wcls->rows};
    a.tokens = S;
    a.qx = s->bqb.qx;
    a.xs = s->bqb.xs;
    if ((rc = batch_product(s, st, "logits", &s->wcls, 1, kEpStore, a))) return rc;
    if (s->sampling) {
        ProfScope p(d, st, "sample");
        launch_sample(sample_args(s, S, s->seq_pos, s->seq_prompt, s->seq_tokens, ctx + 1, nullptr), st);
    } else {
        ProfScope p(d, st, "advance");
        launch_seqs_advance(s->logits, s->wcls->rows, S, s->seq_pos, s->seq_prompt, s->seq_tokens, ctx + 1,
                            (int32_t)(ctx + 1), st);
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? RK_OK : hip_fail(d, e, "stage launch");
}

static int enqueue_rec(rk_stage *s, Rec which, hipStream_t st) {
    switch (which) {
    case kRecToken: return enqueue_token(s, st);
    case kRecSeqs: return enqueue_seqs_step(s, st);
    default: return enqueue_forward(s, st);
    }
}

__global__ void set_ctl_kernel(int32_t *ctl, unsigned long long *amax, int32_t pos, int32_t prompt) {
    ctl[kCtlPos] = pos;
    ctl[kCtlPrompt] = prompt;
    for (int i = 0; i < kArgmaxSlots; i++) amax[i] = 0ull;
}

// The single-sequence entry points run on a stage of one sequence.
static int one_sequence(rk_stage *s, const char *what) {
    if (s->seqs == 1) return RK_OK;
    return fail(s->d, RK_ERR_ARGS, "%s: the stage decodes %d sequences (rk_stage_seqs_*)", what, s->seqs);
}

// Drops the recorded generation steps (they are recorded again on next use).
static void drop_steps(rk_stage *s) {
    if (s->x_token) {
        (void)hipGraphExecDestroy(s->x_token);
        (void)hipGraphDestroy(s->g_token);
        s->x_token = nullptr;
        s->g_token = nullptr;
    }
    if (s->x_seqs) {
        (void)hipGraphExecDestroy(s->x_seqs);
        (void)hipGraphDestroy(s->g_seqs);
        s->x_seqs = nullptr;
        s->g_seqs = nullptr;
    }
}

static bool valid_mat(const rk_matrix *m, rk_device *d, int64_t rows, int64_t cols) {
    return m && m->d == d && (m->kind == RK_Q8 || m->kind == RK_Q4) && m->rows == rows && m->cols == cols;
}

}  // namespace rk

using namespace rk;

extern "C" {

int rk_stage_new(rk_device *d, const rk_stage_config *c, const rk_stage_layer *layers, int32_t n_layers,
                 const float *rope_cos, const float *rope_sin, rk_stage **out) {
    if (!d || !c || !out || n_layers <= 0 || !layers || !rope_cos || !rope_sin)
        return fail(d, RK_ERR_ARGS, "rk_stage_new: bad arguments");
    *out = nullptr;
    const int hs = c->head_dim > 0 ? c->head_dim : (c->heads > 0 ? c->dim / c->heads : 0);
    if (c->dim > kMaxNormCols) return fail(d, RK_ERR_UNSUPPORTED, "rk_stage_new: dim %d beyond %d", c->dim, kMaxNormCols);
    if (c->dim <= 0 || c->hidden <= 0 || c->heads <= 0 || c->kv_heads <= 0 || hs <= 0 || hs % 2 != 0 ||
        c->heads % c->kv_heads != 0 || c->ctx <= 0 || c->dim % 32 != 0 || c->hidden % 32 != 0 ||
        (c->heads * hs) % 32 != 0)
        return fail(d, RK_ERR_ARGS, "rk_stage_new: config out of range");
    // The values kernel keeps a head's weights and a chunk of products in LDS.
    if (c->ctx > att_values_max_ctx())
        return fail(d, RK_ERR_UNSUPPORTED, "rk_stage_new: ctx %d beyond %d", c->ctx, att_values_max_ctx());
    const int qdim = c->heads * hs, kvdim = c->kv_heads * hs;
    const int seqs = std::max(1, c->seqs);
    if (seqs > 256) return fail(d, RK_ERR_ARGS, "rk_stage_new: %d sequences (at most 256)", seqs);
    bool any_moe = false;
    for (int i = 0; i < n_layers; i++) {
        const rk_stage_layer &L = layers[i];
        const bool moe = L.moe != nullptr;
        any_moe = any_moe || moe;
        if (!valid_mat(L.wq, d, qdim, c->dim) || !valid_mat(L.wk, d, kvdim, c->dim) ||
            !valid_mat(L.wv, d, kvdim, c->dim) || !valid_mat(L.wo, d, c->dim, qdim) ||
            (!moe && (!valid_mat(L.w1, d, c->hidden, c->dim) || !valid_mat(L.w3, d, c->hidden, c->dim) ||
                      !valid_mat(L.w2, d, c->dim, c->hidden))))
            return fail(d, RK_ERR_ARGS, "rk_stage_new: layer %d: a matrix is missing, of another shape or device, "
                                        "or not Q8/Q4", i);
        if (moe && (L.moe->d != d || L.moe->dim != c->dim))
            return fail(d, RK_ERR_ARGS, "rk_stage_new: layer %d: its experts take %d values on another device or width",
                        i, (int)L.moe->dim);
        if (!moe && L.w1->kind != L.w3->kind)
            return fail(d, RK_ERR_UNSUPPORTED, "rk_stage_new: layer %d: W1 and W3 differ in format", i);
        if (!L.rms_att || !L.rms_ffn || (c->qkv_bias && (!L.bq || !L.bk || !L.bv)) ||
            (c->qk_norm && (!L.q_norm || !L.k_norm)))
            return fail(d, RK_ERR_ARGS, "rk_stage_new: layer %d: a vector is missing", i);
    }
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    rk_stage *s = new rk_stage();
    s->d = d;
    s->c = *c;
    s->hs = hs;
    s->qdim = qdim;
    s->kvdim = kvdim;
    s->half = hs / 2;
    s->seqs = seqs;
    s->layers.assign(layers, layers + n_layers);
    s->smp_t.assign(seqs, 0.0f);
    // Layout: sizes in bytes, each 256-byte aligned.
    const int64_t ctx = c->ctx;
    const int64_t widest = std::max<int64_t>(std::max<int64_t>(c->dim, qdim), c->hidden);
    int64_t at = 0;
    std::vector<std::pair<void **, int64_t>> plan;
    auto take = [&](void **p, int64_t n) { plan.push_back({p, n}); };
    take((void **)&s->x, 4 * c->dim);
    take((void **)&s->xb, 4 * widest);
    take((void **)&s->q, 4 * qdim);
    take((void **)&s->k, 4 * kvdim);
    take((void **)&s->v, 4 * kvdim);
    take((void **)&s->att, 4 * c->heads * ctx);
    take((void **)&s->att_out, 4 * qdim);
    take((void **)&s->h, 4 * c->hidden);
    take((void **)&s->cos_t, 4 * ctx * s->half);
    take((void **)&s->sin_t, 4 * ctx * s->half);
    take((void **)&s->amax, 8 * kArgmaxSlots);
    take((void **)&s->ctl, 4 * kCtlWords);
    take((void **)&s->tokens, 4 * (ctx + 1));
    take((void **)&s->qx, widest);
    take((void **)&s->xs, 4 * (widest / 32));
    take((void **)&s->xsum, 4 * (widest / 32));
    for (QScratch *q : {&s->qa, &s->qb}) {
        take((void **)&q->qx, widest);
        take((void **)&q->xs, 4 * (widest / 32));
        take((void **)&q->xsum, 4 * (widest / 32));
    }
    take((void **)&s->rms_final, 4 * c->dim);
    take((void **)&s->seq_pos, 4 * seqs);
    take((void **)&s->seq_prompt, 4 * seqs);
    take((void **)&s->seq_tokens, 4 * seqs * (ctx + 1));
    take((void **)&s->smp_temp, 4 * seqs);
    take((void **)&s->smp_state, 8 * seqs);
    take((void **)&s->smp_part, 4 * seqs * sample_parts());
    take((void **)&s->sync, 8 * kSyncWords);
    // the MoE layers' shared scratch, for the largest batch the stage runs
    if (any_moe) {
        s->moe_cap = batch_cap(*c, seqs);
        int64_t mb = 0;
        for (int i = 0; i < n_layers; i++)
            if (layers[i].moe) mb = std::max(mb, moe_scratch_layout(layers[i].moe, s->moe_cap, nullptr, nullptr));
        take((void **)&s->moe_mem, mb);
        take((void **)&s->moe_stat, 16);
        for (int i = 0; i < n_layers; i++)
            if (layers[i].moe) s->moe_sync_stride = std::max(s->moe_sync_stride, moe_sync_words(layers[i].moe));
        take((void **)&s->moe_sync, 8 * s->moe_sync_stride * n_layers);
    }
    s->ld.resize(n_layers);
    const int64_t bias_n = c->qkv_bias ? qdim + 2 * kvdim : 0;
    for (int i = 0; i < n_layers; i++) {
        rk_stage::LayerDev &D = s->ld[i];
        D = rk_stage::LayerDev{};
        take((void **)&D.rms_att, 4 * c->dim);
        take((void **)&D.rms_ffn, 4 * c->dim);
        if (bias_n) take((void **)&D.bias, 4 * bias_n);
        if (c->qk_norm) {
            take((void **)&D.q_norm, 4 * hs);
            take((void **)&D.k_norm, 4 * hs);
        }
        take((void **)&D.keys, 4 * seqs * ctx * kvdim);  // [seqs][ctx][kv_dim]
        take((void **)&D.vals, 4 * seqs * ctx * kvdim);
    }
    for (auto &pl : plan) at += (pl.second + 255) & ~(int64_t)255;
    int rc = dev_alloc(d, (void **)&s->mem, (size_t)at, "stage");
    if (rc) {
        delete s;
        return rc;
    }
    s->bytes = at;
    at = 0;
    for (auto &pl : plan) {
        *pl.first = s->mem + at;
        at += (pl.second + 255) & ~(int64_t)255;
    }
    auto cleanup = [&](int code) {
        (void)hipFree(s->mem);
        if (s->h_x) (void)hipHostFree(s->h_x);
        if (s->h_ctl) (void)hipHostFree(s->h_ctl);
        if (s->h_seq) (void)hipHostFree(s->h_seq);
        delete s;
        return code;
    };
    hipError_t e = hipMemsetAsync(s->mem, 0, (size_t)s->bytes, d->stream);
    auto up = [&](void *dst, const void *src, int64_t bytes) {
        if (e == hipSuccess && bytes > 0) e = hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyHostToDevice, d->stream);
    };
    up(s->cos_t, rope_cos, 4 * ctx * s->half);
    up(s->sin_t, rope_sin, 4 * ctx * s->half);
    for (int i = 0; i < n_layers; i++) {
        const rk_stage_layer &L = layers[i];
        rk_stage::LayerDev &D = s->ld[i];
        up(D.rms_att, L.rms_att, 4 * c->dim);
        up(D.rms_ffn, L.rms_ffn, 4 * c->dim);
        if (bias_n) {
            up(D.bias, L.bq, 4 * qdim);
            up(D.bias + qdim, L.bk, 4 * kvdim);
            up(D.bias + qdim + kvdim, L.bv, 4 * kvdim);
        }
        if (c->qk_norm) {
            up(D.q_norm, L.q_norm, 4 * hs);
            up(D.k_norm, L.k_norm, 4 * hs);
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return cleanup(hip_fail(d, e, "stage upload"));
    }
    if ((e = hipHostMalloc((void **)&s->h_x, (size_t)4 * kForwardBatch * c->dim, hipHostMallocDefault)) !=
            hipSuccess ||
        (e = hipHostMalloc((void **)&s->h_ctl, (size_t)4 * (ctx + 1 + kCtlWords), hipHostMallocDefault)) !=
            hipSuccess ||
        (e = hipHostMalloc((void **)&s->h_seq, (size_t)4 * seqs * (ctx + 3), hipHostMallocDefault)) != hipSuccess) {
        (void)hipGetLastError();
        return cleanup(hip_fail(d, e, "stage staging"));
    }
    add_used(d, s->bytes);
    *out = s;
    return RK_OK;
}

int rk_stage_forward(rk_stage *s, float *xs, int32_t pos, int32_t tokens) {
    if (!s) return RK_ERR_ARGS;
    rk_device *d = s->d;
    if (int rc = one_sequence(s, "rk_stage_forward")) return rc;
    if (tokens < 0 || (tokens > 0 && !xs) || pos < 0 || (int64_t)pos + tokens > s->c.ctx)
        return fail(d, RK_ERR_ARGS, "gpu stage: positions [%d, %d) outside the context of %d", pos, pos + tokens,
                    s->c.ctx);
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    hipStream_t st = d->stream;
    const int dim = s->c.dim;
    if (tokens > 1) {
        // several tokens: the batched path (same bits as one at a time)
        int rc = batch_alloc(s);
        if (rc) return rc;
        for (int start = 0; start < tokens; start += s->bcap) {
            const int n = std::min(s->bcap, tokens - start);
            HIP_TRY(d, hipMemcpyAsync(s->bx, xs + (int64_t)start * dim, (size_t)n * dim * 4, hipMemcpyHostToDevice, st),
                    "stage input");
            if ((rc = enqueue_forward_batch(s, st, n, at_pos(pos + start)))) return rc;
            HIP_TRY(d, hipMemcpyAsync(xs + (int64_t)start * dim, s->bx, (size_t)n * dim * 4, hipMemcpyDeviceToHost, st),
                    "stage output");
            HIP_TRY(d, hipStreamSynchronize(st), "stage submit");
        }
        return RK_OK;
    }
    for (int start = 0; start < tokens; start += kForwardBatch) {
        const int n = std::min(kForwardBatch, tokens - start);
        memcpy(s->h_x, xs + (int64_t)start * dim, (size_t)n * dim * 4);
        for (int t = 0; t < n; t++) {
            HIP_TRY(d, hipMemcpyAsync(s->x, s->h_x + (int64_t)t * dim, (size_t)dim * 4, hipMemcpyHostToDevice, st),
                    "stage input");
            hipLaunchKernelGGL(set_ctl_kernel, dim3(1), dim3(1), 0, st, s->ctl, s->amax, pos + start + t, 0);
            int rc = run_once(s, kRecLayers);
            if (rc) return rc;
            HIP_TRY(d, hipMemcpyAsync(s->h_x + (int64_t)t * dim, s->x, (size_t)dim * 4, hipMemcpyDeviceToHost, st),
                    "stage output");
        }
        HIP_TRY(d, hipStreamSynchronize(st), "stage submit");
        memcpy(xs + (int64_t)start * dim, s->h_x, (size_t)n * dim * 4);
    }
    return tokens > 0 ? sync_check(s, "stage submit") : RK_OK;
}

int64_t rk_stage_bytes(const rk_stage *s) { return s ? s->bytes : -1; }

int rk_stage_free(rk_stage *s) {
    if (!s) return RK_ERR_ARGS;
    rk_device *d = s->d;
    Hold hold(d->gate);
    (void)hipSetDevice(d->index);
    (void)hipStreamSynchronize(d->stream);
    if (s->x_layers) (void)hipGraphExecDestroy(s->x_layers);
    if (s->g_layers) (void)hipGraphDestroy(s->g_layers);
    if (s->x_token) (void)hipGraphExecDestroy(s->x_token);
    if (s->g_token) (void)hipGraphDestroy(s->g_token);
    if (s->x_seqs) (void)hipGraphExecDestroy(s->x_seqs);
    if (s->g_seqs) (void)hipGraphDestroy(s->g_seqs);
    (void)hipFree(s->mem);
    (void)hipFree(s->bmem);
    (void)hipFree(s->logits);
    if (s->h_x) (void)hipHostFree(s->h_x);
    if (s->h_ctl) (void)hipHostFree(s->h_ctl);
    if (s->h_seq) (void)hipHostFree(s->h_seq);
    if (s->h_logits) (void)hipHostFree(s->h_logits);
    (void)hipGetLastError();
    add_used(d, -s->bytes);
    delete s;
    return RK_OK;
}

int rk_stage_set_head(rk_stage *s, rk_matrix *embed, rk_matrix *wcls, const float *rms_final) {
    if (!s) return RK_ERR_ARGS;
    rk_device *d = s->d;
    if (!embed || !wcls || !rms_final || embed->d != d || wcls->d != d || embed->cols != s->c.dim ||
        wcls->cols != s->c.dim || embed->rows != wcls->rows ||
        (embed->kind != RK_Q8 && embed->kind != RK_Q4) || (wcls->kind != RK_Q8 && wcls->kind != RK_Q4))
        return fail(d, RK_ERR_ARGS, "rk_stage_set_head: embedding or classifier of the wrong shape or format");
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    drop_steps(s);
    // logits of every sequence, [seqs][vocab], then the sampler's terms
    // [seqs][stride] (16-byte aligned)
    const int64_t nl = wcls->rows * s->seqs;
    const int64_t nl_pad = (nl + 63) & ~(int64_t)63;
    const int64_t ndev = nl_pad + s->seqs * sample_terms_stride(wcls->rows);
    if (s->logits && (nl > s->logits_n || ndev > s->logits_dev)) {
        HIP_TRY(d, hipStreamSynchronize(d->stream), "logits");
        (void)hipFree(s->logits);
        (void)hipHostFree(s->h_logits);
        s->logits = nullptr;
        s->h_logits = nullptr;
        s->bytes -= 4 * s->logits_dev;
        add_used(d, -4 * s->logits_dev);
        s->logits_n = 0;
        s->logits_dev = 0;
    }
    if (!s->logits) {
        int rc = dev_alloc(d, (void **)&s->logits, (size_t)4 * ndev, "logits");
        if (rc) return rc;
        hipError_t e = hipHostMalloc((void **)&s->h_logits, (size_t)4 * nl, hipHostMallocDefault);
        if (e != hipSuccess) {
            (void)hipFree(s->logits);
            s->logits = nullptr;
            return hip_fail(d, e, "logits staging");
        }
        s->logits_n = nl;
        s->logits_dev = ndev;
        s->bytes += 4 * ndev;
        add_used(d, 4 * ndev);
    }
    s->smp_terms = s->logits + nl_pad;
    HIP_TRY(d, hipMemcpyAsync(s->rms_final, rms_final, (size_t)4 * s->c.dim, hipMemcpyHostToDevice, d->stream),
            "head upload");
    HIP_TRY(d, hipStreamSynchronize(d->stream), "head upload");
    s->embed = embed;
    s->wcls = wcls;
    return RK_OK;
}

int rk_stage_generate_start(rk_stage *s, const int32_t *prompt, int32_t n_prompt) {
    if (!s) return RK_ERR_ARGS;
    rk_device *d = s->d;
    if (int rc = one_sequence(s, "rk_stage_generate")) return rc;
    if (!s->embed) return fail(d, RK_ERR_ARGS, "rk_stage_generate: the stage has no head");
    if (!prompt || n_prompt <= 0 || n_prompt > s->c.ctx)
        return fail(d, RK_ERR_ARGS, "rk_stage_generate: prompt of %d tokens for a context of %d", n_prompt, s->c.ctx);
    const int64_t vocab = s->embed->rows;
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= vocab)
            return fail(d, RK_ERR_ARGS, "rk_stage_generate: token %d out of range", prompt[i]);
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    HIP_TRY(d, hipStreamSynchronize(d->stream), "generate start");
    memcpy(s->h_ctl, prompt, (size_t)n_prompt * 4);
    HIP_TRY(d, hipMemcpyAsync(s->tokens, s->h_ctl, (size_t)n_prompt * 4, hipMemcpyHostToDevice, d->stream),
            "prompt upload");
    hipLaunchKernelGGL(set_ctl_kernel, dim3(1), dim3(1), 0, d->stream, s->ctl, s->amax, 0, n_prompt);
    HIP_TRY(d, hipGetLastError(), "generate start");
    s->prompt_n = n_prompt;
    HIP_TRY(d, hipStreamSynchronize(d->stream), "generate start");
    return RK_OK;
}

int rk_stage_generate_run(rk_stage *s, int32_t positions, float *logits) {
    if (!s || positions < 0) return RK_ERR_ARGS;
    rk_device *d = s->d;
    if (int rc = one_sequence(s, "rk_stage_generate")) return rc;
    if (!s->embed) return fail(d, RK_ERR_ARGS, "rk_stage_generate: the stage has no head");
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    // The device holds the position; the host checks the context bound.
    int32_t pos = 0;
    HIP_TRY(d, hipMemcpyAsync(s->h_ctl + s->c.ctx + 1, s->ctl + kCtlPos, 4, hipMemcpyDeviceToHost, d->stream),
            "position");
    HIP_TRY(d, hipStreamSynchronize(d->stream), "position");
    pos = s->h_ctl[s->c.ctx + 1];
    if ((int64_t)pos + positions > s->c.ctx)
        return fail(d, RK_ERR_ARGS, "rk_stage_generate: positions [%d, %d) outside the context of %d", pos,
                    pos + positions, s->c.ctx);
    const int64_t vocab = s->wcls->rows;
    // Prompt positions before the last compute no logits: with no logits
    // asked for, two or more of them go through the batched path (their
    // embeddings, the layers; the same cache entries), then the position
    // moves on.
    if (!logits && pos + 2 < s->prompt_n && positions >= 2) {
        int rc = batch_alloc(s);
        if (rc) return rc;
        hipStream_t st = d->stream;
        int left = std::min(positions, s->prompt_n - 1 - pos);
        positions -= left;
        while (left > 0) {
            const int n = std::min(left, s->bcap);
            {
                ProfScope p(d, st, "embed");
                launch_embed_rows(s->embed->w, s->embed->scales, s->embed->kind == RK_Q4, s->tokens, pos, n, s->c.dim,
                                  s->bx, st);
            }
            if ((rc = enqueue_forward_batch(s, st, n, at_pos(pos)))) return rc;
            pos += n;
            left -= n;
            hipLaunchKernelGGL(set_ctl_kernel, dim3(1), dim3(1), 0, st, s->ctl, s->amax, pos, s->prompt_n);
            HIP_TRY(d, hipGetLastError(), "generate prefill");
        }
    }
    for (int32_t i = 0; i < positions; i++) {
        int rc = run_once(s, kRecToken);
        if (rc) return rc;
        if (logits) {
            HIP_TRY(d, hipMemcpyAsync(s->h_logits, s->logits, (size_t)vocab * 4, hipMemcpyDeviceToHost, d->stream),
                    "logits");
            HIP_TRY(d, hipStreamSynchronize(d->stream), "generate step");
            memcpy(logits + (int64_t)i * vocab, s->h_logits, (size_t)vocab * 4);
        }
    }
    HIP_TRY(d, hipStreamSynchronize(d->stream), "generate run");
    return sync_check(s, "generate run");
}

int rk_stage_generate_tokens(rk_stage *s, int32_t from, int32_t n, int32_t *out) {
    if (!s || !out || from < 0 || n < 0 || (int64_t)from + n > s->c.ctx + 1) return RK_ERR_ARGS;
    rk_device *d = s->d;
    if (int rc = one_sequence(s, "rk_stage_generate_tokens")) return rc;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    HIP_TRY(d, hipStreamSynchronize(d->stream), "tokens");
    HIP_TRY(d, hipMemcpyAsync(out, s->tokens + from, (size_t)n * 4, hipMemcpyDeviceToHost, d->stream), "tokens");
    HIP_TRY(d, hipStreamSynchronize(d->stream), "tokens");
    return RK_OK;
}

int rk_stage_generate(rk_stage *s, const int32_t *prompt, int32_t n_prompt, int32_t steps, int32_t *out) {
    if (!s || steps < 0 || (steps > 0 && !out)) return RK_ERR_ARGS;
    int rc = rk_stage_generate_start(s, prompt, n_prompt);
    if (rc || steps == 0) return rc;
    if ((rc = rk_stage_generate_run(s, n_prompt + steps - 1, nullptr))) return rc;
    return rk_stage_generate_tokens(s, n_prompt, steps, out);
}

int rk_stage_seqs_start(rk_stage *s, const int32_t *prompts, const int32_t *lens) {
    if (!s) return RK_ERR_ARGS;
    rk_device *d = s->d;
    if (!s->embed) return fail(d, RK_ERR_ARGS, "rk_stage_seqs_start: the stage has no head");
    if (!prompts || !lens) return fail(d, RK_ERR_ARGS, "rk_stage_seqs_start: null argument");
    const int S = s->seqs;
    const int64_t ctx = s->c.ctx, vocab = s->embed->rows;
    int64_t total = 0;
    for (int z = 0; z < S; z++) {
        if (lens[z] <= 0 || lens[z] > ctx)
            return fail(d, RK_ERR_ARGS, "rk_stage_seqs_start: sequence %d: prompt of %d tokens for a context of %lld", z,
                        lens[z], (long long)ctx);
        for (int i = 0; i < lens[z]; i++)
            if (prompts[total + i] < 0 || prompts[total + i] >= vocab)
                return fail(d, RK_ERR_ARGS, "rk_stage_seqs_start: sequence %d: token %d out of range", z,
                            prompts[total + i]);
        total += lens[z];
    }
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    hipStream_t st = d->stream;
    HIP_TRY(d, hipStreamSynchronize(st), "seqs start");
    int rc = batch_alloc(s);
    if (rc) return rc;
    // tokens [S][ctx+1] (each prompt at the start of its row), then the
    // positions (each prompt's last) and the prompt lengths
    int32_t *h = s->h_seq;
    memset(h, 0, (size_t)4 * S * (ctx + 1));
    int64_t at = 0;
    for (int z = 0; z < S; z++) {
        memcpy(h + z * (ctx + 1), prompts + at, (size_t)4 * lens[z]);
        at += lens[z];
        h[S * (ctx + 1) + z] = lens[z] - 1;
        h[S * (ctx + 1) + S + z] = lens[z];
    }
    HIP_TRY(d, hipMemcpyAsync(s->seq_tokens, h, (size_t)4 * S * (ctx + 1), hipMemcpyHostToDevice, st), "prompts");
    HIP_TRY(d, hipMemcpyAsync(s->seq_pos, h + S * (ctx + 1), (size_t)4 * S, hipMemcpyHostToDevice, st), "positions");
    HIP_TRY(d, hipMemcpyAsync(s->seq_prompt, h + S * (ctx + 1) + S, (size_t)4 * S, hipMemcpyHostToDevice, st),
            "prompt lengths");
    // every prompt position but the last: each sequence's batched prefill
    // into its own caches (the same bits as one position at a time)
    for (int z = 0; z < S; z++) {
        for (int start = 0; start < lens[z] - 1; start += s->bcap) {
            const int n = std::min(s->bcap, lens[z] - 1 - start);
            {
                ProfScope p(d, st, "embed");
                launch_embed_rows(s->embed->w, s->embed->scales, s->embed->kind == RK_Q4, s->seq_tokens + z * (ctx + 1),
                                  start, n, s->c.dim, s->bx, st);
            }
            BatchPos bp;
            bp.pos0 = start;
            bp.cache0 = (int64_t)z * ctx * s->kvdim;
            if ((rc = enqueue_forward_batch(s, st, n, bp))) return rc;
        }
    }
    HIP_TRY(d, hipStreamSynchronize(st), "seqs prefill");
    s->seq_at.assign(lens, lens + S);
    for (int32_t &p : s->seq_at) p -= 1;
    s->seqs_started = true;
    return RK_OK;
}

int rk_stage_seqs_run(rk_stage *s, int32_t steps, float *logits) {
    if (!s || steps < 0) return RK_ERR_ARGS;
    rk_device *d = s->d;
    if (!s->seqs_started) return fail(d, RK_ERR_ARGS, "rk_stage_seqs_run: no sequences started");
    const int S = s->seqs;
    for (int z = 0; z < S; z++)
        if ((int64_t)s->seq_at[z] + steps > s->c.ctx)
            return fail(d, RK_ERR_ARGS, "rk_stage_seqs_run: sequence %d: positions [%d, %d) outside the context of %d", z,
                        s->seq_at[z], s->seq_at[z] + steps, s->c.ctx);
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    const int64_t n = (int64_t)S * s->wcls->rows;
    for (int32_t i = 0; i < steps; i++) {
        int rc = run_once(s, kRecSeqs);
        if (rc) return rc;
        if (logits) {
            HIP_TRY(d, hipMemcpyAsync(s->h_logits, s->logits, (size_t)n * 4, hipMemcpyDeviceToHost, d->stream),
                    "logits");
            HIP_TRY(d, hipStreamSynchronize(d->stream), "seqs step");
            memcpy(logits + (int64_t)i * n, s->h_logits, (size_t)n * 4);
        }
    }
    HIP_TRY(d, hipStreamSynchronize(d->stream), "seqs run");
    for (int32_t &p : s->seq_at) p += steps;
    return RK_OK;
}

int rk_stage_moe_stats(rk_stage *s, int64_t *selected, int64_t *groupings) {
    if (!s || !selected || !groupings) return RK_ERR_ARGS;
    rk_device *d = s->d;
    *selected = 0;
    *groupings = 0;
    if (!s->moe_stat) return RK_OK;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    unsigned long long v[2] = {0, 0};
    HIP_TRY(d, hipStreamSynchronize(d->stream), "moe stats");
    HIP_TRY(d, hipMemcpy(v, s->moe_stat, 16, hipMemcpyDeviceToHost), "moe stats");
    HIP_TRY(d, hipMemset(s->moe_stat, 0, 16), "moe stats");
    *selected = (int64_t)v[0];
    *groupings = (int64_t)v[1];
    return RK_OK;
}

int rk_stage_sampler(rk_stage *s, int32_t seq, float temperature, uint64_t seed) {
    if (!s) return RK_ERR_ARGS;
    rk_device *d = s->d;
    if (seq < 0 || seq >= s->seqs)
        return fail(d, RK_ERR_ARGS, "rk_stage_sampler: sequence %d of %d", seq, s->seqs);
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    hipStream_t st = d->stream;
    HIP_TRY(d, hipStreamSynchronize(st), "sampler");
    // internal/llm/sample.go:11-16: a zero seed is replaced
    const uint64_t state = seed == 0 ? 0x9e3779b97f4a7c15ull : seed;
    HIP_TRY(d, hipMemcpyAsync(s->smp_temp + seq, &temperature, 4, hipMemcpyHostToDevice, st), "sampler");
    HIP_TRY(d, hipMemcpyAsync(s->smp_state + seq, &state, 8, hipMemcpyHostToDevice, st), "sampler");
    HIP_TRY(d, hipStreamSynchronize(st), "sampler");
    s->smp_t[seq] = temperature;
    // NaN samples, as in the reference (only temperature <= 0 is greedy)
    bool sampling = false;
    for (float t : s->smp_t) sampling = sampling || !(t <= 0.0f);
    if (sampling != s->sampling) {
        drop_steps(s);
        s->sampling = sampling;
    }
    return RK_OK;
}

int rk_stage_seqs_tokens(rk_stage *s, int32_t seq, int32_t from, int32_t n, int32_t *out) {
    if (!s || !out || seq < 0 || seq >= s->seqs || from < 0 || n < 0 || (int64_t)from + n > s->c.ctx + 1)
        return RK_ERR_ARGS;
    rk_device *d = s->d;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    HIP_TRY(d, hipStreamSynchronize(d->stream), "tokens");
    HIP_TRY(d,
            hipMemcpyAsync(out, s->seq_tokens + (int64_t)seq * (s->c.ctx + 1) + from, (size_t)n * 4,
                           hipMemcpyDeviceToHost, d->stream),
            "tokens");
    HIP_TRY(d, hipStreamSynchronize(d->stream), "tokens");
    return RK_OK;
}

}  // extern "C"
