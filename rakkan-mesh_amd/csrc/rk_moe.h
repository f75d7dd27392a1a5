// rk_moe.h — the mixture-of-experts feed-forward's internals, shared by the
// standalone rk_moe_* entry points and the stages that hold MoE layers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rk_runtime.h"

namespace rk {

// Device scratch of one MoE feed-forward over up to `cap` tokens (a stage
// shares one among its MoE layers, which run one after another).
struct MoeScratch {
    int cap = 0;
    int gcap = 0;                  // groups the layout holds: min(experts, cap·topk)
    float *logits = nullptr;       // [cap][experts]
    int32_t *sel = nullptr;        // [cap][topk] selected experts, selection order
    float *wsel = nullptr;         // [cap][topk] their weights
    int32_t *grp = nullptr;        // groups: count, expert[gcap], start[gcap], pairs[gcap], pair list[cap·topk]
    float *gwt = nullptr;          // [cap·topk] the pair list's weights (wsel of each listed pair)
    const void **gptr = nullptr;   // [gcap][6] each group's expert rows: W1, W1 scales, W3, W3 scales, W2, W2 scales
    int8_t *hq = nullptr;          // [cap·topk][hidden] each (token, slot)'s h, quantized
    float *hs = nullptr;
    int32_t *hsum = nullptr;
    float *o = nullptr;            // [cap·topk][dim] each (token, slot)'s W2·h
    // optional: each grouping of several tokens adds its selected experts'
    // count to stat[0] and 1 to stat[1]
    unsigned long long *stat = nullptr;
    // optional: one token's feed-forward in one launch (moe_ffn1_kernel)
    // takes moe_sync_words() hand-off words (zero when made, owned by one
    // layer: every launch on them has the same shape and tags them with
    // that layer's count) and the word a timed-out wait sets
    unsigned long long *sync = nullptr;
    unsigned long long *err = nullptr;
};

}  // namespace rk

// One MoE feed-forward's weights: the router and each expert's W1, W3, W2
// (caller-owned matrices), with device tables of their codes and scales.
struct rk_moe {
    rk_device *d = nullptr;
    rk_matrix *router = nullptr;
    int32_t experts = 0, topk = 0, dim = 0, hidden = 0;
    const uint8_t **w1 = nullptr, **w3 = nullptr, **w2 = nullptr;
    const float **s1 = nullptr, **s3 = nullptr, **s2 = nullptr;
    void *tables = nullptr;
    // scratch of the standalone calls (rk_moe_ffn*), grown to the largest
    // batch: the input, its quantized form, the output, and a MoeScratch
    void *mem = nullptr;
    int64_t bytes = 0;
    int cap = 0;
    float *x = nullptr, *y = nullptr;
    int8_t *qx = nullptr;
    float *xs = nullptr;
    int32_t *xsum = nullptr;
    rk::MoeScratch sc;
};

namespace rk {

// 64-bit words of one layer's hand-off area for the one-token launch (the
// selection's lines, the tagged logits and h blocks, the count words).
int64_t moe_sync_words(const rk_moe *m);

// Bytes of a MoeScratch for `cap` tokens of m; with mem, also lays it out
// there (256-byte aligned pieces). A stage sizes one for the largest of its
// MoE layers.
int64_t moe_scratch_layout(const rk_moe *m, int cap, char *mem, MoeScratch *sc);

// The feed-forward of `tokens` inputs already quantized (qx [tokens][dim]
// codes, xs/xsum [tokens][dim/32]): out = y, or (residual) out =
// Canonical(out + y), rows [tokens][dim]. Enqueue only; it allocates
// nothing, so it may be recorded into a graph.
struct MoeNext;
int enqueue_moe_q(rk_moe *m, const MoeScratch &sc, const int8_t *qx, const float *xs, const int32_t *xsum,
                  int tokens, float *out, bool residual, hipStream_t s, const MoeNext *next = nullptr);

// The next product's input, formed after the sum into the residual:
// RMSNorm of each new row with norm_w, quantized into qx/xs/xsum.
struct MoeNext {
    const float *norm_w;
    float recip_n, eps;
    int8_t *qx;
    float *xs;
    int32_t *xsum;
};

// The same from f32 inputs x [tokens][dim]: RMSNorm'd with norm_w (recip_n
// = 1/dim, eps) or, norm_w null, taken as given, and quantized into qx/xs/
// xsum (which the experts' products then read). With `next` (residual only,
// several tokens), the sum's launch also forms the next product's input.
int enqueue_moe_x(rk_moe *m, const MoeScratch &sc, const float *x, const float *norm_w, float recip_n, float eps,
                  int tokens, int8_t *qx, float *xs, int32_t *xsum, float *out, bool residual, hipStream_t s,
                  const MoeNext *next = nullptr);

}  // namespace rk
