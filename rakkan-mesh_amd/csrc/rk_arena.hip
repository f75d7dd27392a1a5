// rk_arena.hip — arenas, vectors and batches: the device memory and the
// recorded operations the llama stage runs on (internal/gpu/batch.go). Ops
// take word offsets into the arena as the Go API does; every span is checked
// against the arena (or vectors) before a kernel touches it. Ops are
// enqueued on the device's stream as they are recorded; nothing is visible
// to the host until rk_batch_submit, which waits and delivers the reads.
#include <algorithm>
#include <cstring>

#include "rk_layer.h"
#include "rk_mx.h"
#include "rk_runtime.h"

// internal/gpu/batch.go:12-20 Arena.
struct rk_arena {
    rk_device *d = nullptr;
    int64_t words = 0, staging_words = 0;
    float *buf = nullptr;       // device words
    float *staging = nullptr;   // pinned host words
    int64_t qx_off = -1, xs_off = -1;
    // The quantized input of products (kept here, 16-byte aligned, rather
    // than in the reserved words: the kernels read it as 128-bit vectors).
    // Quantize and QuantizeFP8 also leave their result in the reserved
    // words, in the reference's layout, for callers that read it back.
    int8_t *qx = nullptr;
    float *xs = nullptr;
    int32_t *xsum = nullptr;
    int64_t bytes = 0;
};

// internal/gpu/batch.go:113-124 Batch.
struct rk_batch {
    rk_arena *a = nullptr;
    int64_t staged = 0;
    struct PendingRead {
        float *dst;
        int64_t at, n;
    };
    std::vector<PendingRead> reads;
    int err = RK_OK;
};

namespace rk {

static int latch(rk_batch *b, int code) {
    if (b->err == RK_OK) b->err = code;
    return b->err;
}

// Device pointer of words [off, off+n) of the arena, or null (and the error
// latched) if the span leaves it.
static float *span(rk_batch *b, int64_t off, int64_t n, const char *what) {
    rk_arena *a = b->a;
    if (off < 0 || n < 0 || off > a->words || n > a->words - off) {
        latch(b, fail(a->d, RK_ERR_ARGS, "gpu: %s words [%lld, %lld) outside the arena of %lld", what, (long long)off,
                      (long long)(off + n), (long long)a->words));
        return nullptr;
    }
    return a->buf + off;
}

static const float *vspan(rk_batch *b, rk_vectors *v, int64_t off, int64_t n, const char *what) {
    if (!v || v->d != b->a->d || off < 0 || n < 0 || off > v->n || n > v->n - off) {
        latch(b, fail(b->a->d, RK_ERR_ARGS, "gpu: %s outside its vectors", what));
        return nullptr;
    }
    return v->buf + off;
}

static int launched(rk_batch *b, const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return latch(b, hip_fail(b->a->d, e, what));
    return RK_OK;
}

}  // namespace rk

using namespace rk;

extern "C" {

int rk_arena_new(rk_device *d, int64_t words, int64_t staging_words, rk_arena **out) {
    if (!d || !out || words < 0 || staging_words < 0) return fail(d, RK_ERR_ARGS, "rk_arena_new: bad arguments");
    *out = nullptr;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    rk_arena *a = new rk_arena();
    a->d = d;
    a->words = words;
    a->staging_words = staging_words;
    int rc = dev_alloc(d, (void **)&a->buf, (size_t)(words > 0 ? words : 1) * 4, "arena");
    if (rc) {
        delete a;
        return rc;
    }
    hipError_t e = hipHostMalloc((void **)&a->staging, (size_t)(staging_words > 0 ? staging_words : 1) * 4,
                                 hipHostMallocDefault);
    if (e != hipSuccess) {
        (void)hipFree(a->buf);
        delete a;
        return hip_fail(d, e, "arena staging");
    }
    a->bytes = (words > 0 ? words : 1) * 4;
    add_used(d, a->bytes);
    *out = a;
    return RK_OK;
}

int rk_arena_set_quant_scratch(rk_arena *a, int64_t qx_off, int64_t xs_off) {
    if (!a) return RK_ERR_ARGS;
    rk_device *d = a->d;
    if (qx_off < 0 || xs_off < 0 || qx_off >= a->words || xs_off >= a->words)
        return fail(d, RK_ERR_ARGS, "rk_arena_set_quant_scratch: offsets outside the arena");
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    if (!a->qx) {
        int rc;
        if ((rc = dev_alloc(d, (void **)&a->qx, kMaxCols, "quant scratch")) ||
            (rc = dev_alloc(d, (void **)&a->xs, 4 * (kMaxCols / 32), "quant scratch")) ||
            (rc = dev_alloc(d, (void **)&a->xsum, 4 * (kMaxCols / 32), "quant scratch"))) {
            (void)hipFree(a->qx);
            (void)hipFree(a->xs);
            a->qx = nullptr;
            a->xs = nullptr;
            return rc;
        }
        const int64_t extra = kMaxCols + 8 * (kMaxCols / 32);
        a->bytes += extra;
        add_used(d, extra);
    }
    a->qx_off = qx_off;
    a->xs_off = xs_off;
    return RK_OK;
}

int64_t rk_arena_bytes(const rk_arena *a) { return a ? a->bytes : -1; }

int rk_arena_device_ptr(rk_arena *a, int64_t off, void **dptr) {
    if (!a || !dptr || off < 0 || off > a->words) return RK_ERR_ARGS;
    *dptr = a->buf + off;
    return RK_OK;
}

int rk_arena_free(rk_arena *a) {
    if (!a) return RK_ERR_ARGS;
    rk_device *d = a->d;
    Hold hold(d->gate);
    (void)hipSetDevice(d->index);
    (void)hipStreamSynchronize(d->stream);
    (void)hipFree(a->buf);
    (void)hipFree(a->qx);
    (void)hipFree(a->xs);
    (void)hipFree(a->xsum);
    (void)hipHostFree(a->staging);
    add_used(d, -a->bytes);
    delete a;
    return RK_OK;
}

int rk_vectors_upload(rk_device *d, const float *v, int64_t n, rk_vectors **out) {
    if (!d || !out || n < 0 || (n > 0 && !v)) return fail(d, RK_ERR_ARGS, "rk_vectors_upload: bad arguments");
    *out = nullptr;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    rk_vectors *vs = new rk_vectors();
    vs->d = d;
    vs->n = n;
    int rc = dev_alloc(d, (void **)&vs->buf, (size_t)(n > 0 ? n : 1) * 4, "vectors");
    if (rc) {
        delete vs;
        return rc;
    }
    if (n > 0) {
        hipError_t e = hipMemcpy(vs->buf, v, (size_t)n * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(vs->buf);
            delete vs;
            return hip_fail(d, e, "vectors upload");
        }
    }
    vs->bytes = (n > 0 ? n : 1) * 4;
    add_used(d, vs->bytes);
    *out = vs;
    return RK_OK;
}

int rk_vectors_free(rk_vectors *v) {
    if (!v) return RK_ERR_ARGS;
    rk_device *d = v->d;
    Hold hold(d->gate);
    (void)hipSetDevice(d->index);
    (void)hipStreamSynchronize(d->stream);
    (void)hipFree(v->buf);
    add_used(d, -v->bytes);
    delete v;
    return RK_OK;
}

int rk_batch_begin(rk_arena *a, rk_batch **out) {
    if (!a || !out) return RK_ERR_ARGS;
    a->d->gate.acquire();  // released by rk_batch_submit
    rk_batch *b = new rk_batch();
    b->a = a;
    if (hipSetDevice(a->d->index) != hipSuccess) {
        (void)hipGetLastError();
        latch(b, fail(a->d, RK_ERR_HIP, "hipSetDevice"));
    }
    *out = b;
    return RK_OK;
}

int rk_batch_write(rk_batch *b, int64_t off, const float *data, int64_t n) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    if (n == 0) return RK_OK;
    if (!data) return latch(b, fail(b->a->d, RK_ERR_ARGS, "rk_batch_write: null data"));
    rk_arena *a = b->a;
    if (b->staged + n > a->staging_words)
        return latch(b, fail(a->d, RK_ERR_ARGS, "gpu: batch moves more than its staging holds"));
    float *dst = span(b, off, n, "write");
    if (!dst) return b->err;
    float *st = a->staging + b->staged;
    memcpy(st, data, (size_t)n * 4);
    b->staged += n;
    hipError_t e = hipMemcpyAsync(dst, st, (size_t)n * 4, hipMemcpyHostToDevice, a->d->stream);
    if (e != hipSuccess) return latch(b, hip_fail(a->d, e, "batch write"));
    return RK_OK;
}

int rk_batch_read(rk_batch *b, int64_t off, float *dst, int64_t n) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    if (n == 0) return RK_OK;
    if (!dst) return latch(b, fail(b->a->d, RK_ERR_ARGS, "rk_batch_read: null destination"));
    rk_arena *a = b->a;
    if (b->staged + n > a->staging_words)
        return latch(b, fail(a->d, RK_ERR_ARGS, "gpu: batch moves more than its staging holds"));
    const float *src = span(b, off, n, "read");
    if (!src) return b->err;
    float *st = a->staging + b->staged;
    hipError_t e = hipMemcpyAsync(st, src, (size_t)n * 4, hipMemcpyDeviceToHost, a->d->stream);
    if (e != hipSuccess) return latch(b, hip_fail(a->d, e, "batch read"));
    b->reads.push_back({dst, b->staged, n});
    b->staged += n;
    return RK_OK;
}

// internal/gpu/batch.go:212-269 MatVecs: the input quantized once into the
// arena's scratch, each matrix's rows to its own offset.
int rk_batch_matvecs(rk_batch *b, int32_t n, rk_matrix *const *ms, const int64_t *out_offs, int64_t in_off) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    if (n <= 0) return RK_OK;
    rk_arena *a = b->a;
    rk_device *d = a->d;
    if (!ms || !out_offs) return latch(b, fail(d, RK_ERR_ARGS, "rk_batch_matvecs: null arguments"));
    const int64_t cols = ms[0] ? ms[0]->cols : 0;
    std::vector<float *> outs(n);
    bool quantized = false;
    for (int i = 0; i < n; i++) {
        rk_matrix *m = ms[i];
        if (!m || m->d != d) return latch(b, fail(d, RK_ERR_ARGS, "gpu: matrix on another device"));
        if (m->cols != cols) return latch(b, fail(d, RK_ERR_ARGS, "gpu: products of one input need one width"));
        if (m->kind < RK_F32 || m->kind > RK_FP4)
            return latch(b, fail(d, RK_ERR_UNSUPPORTED, "rk_batch_matvecs: format %d has no kernel in this build",
                                 m->kind));
        if (!(outs[i] = span(b, out_offs[i], m->rows, "product output"))) return b->err;
        quantized = quantized || (m->kind != RK_F32 && m->kind != RK_BF16);
    }
    if (int rc = mixed_inputs(d, n, ms)) return latch(b, rc);
    // internal/gpu/batch.go:240-245: only a quantized product needs the scratch
    if (quantized && a->qx_off < 0)
        return latch(b, fail(d, RK_ERR_ARGS, "gpu: arena has no scratch for quantized inputs"));
    const float *x = span(b, in_off, cols, "product input");
    if (!x) return b->err;
    int rc = enqueue_matvecs(d, n, ms, outs.data(), x, cols, QScratch{a->qx, a->xs, a->xsum}, d->stream);
    return rc ? latch(b, rc) : RK_OK;
}

// internal/gpu/batch.go:277-280 Quantize: the input's Q8_0 form into the
// products' scratch, and, as the reference leaves it in the arena, its
// codes four a word (little-endian, code j in byte j) at qx_off and its
// block scales at xs_off (internal/gpu/kernels.go:323-353).
int rk_batch_quantize(rk_batch *b, int64_t in, int64_t n) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    rk_arena *a = b->a;
    if (a->qx_off < 0) return latch(b, fail(a->d, RK_ERR_ARGS, "gpu: arena has no scratch for quantized inputs"));
    if (n % 32 != 0 || n > kMaxCols) return latch(b, fail(a->d, RK_ERR_ARGS, "gpu: quantize of %lld floats", (long long)n));
    const float *x = span(b, in, n, "quantize input");
    float *qw = x ? span(b, a->qx_off, n / 4, "quantized codes") : nullptr;
    float *sw = qw ? span(b, a->xs_off, n / 32, "quantized scales") : nullptr;
    if (!sw) return b->err;
    hipStream_t s = a->d->stream;
    {
        ProfScope p(a->d, s, "quantize_acts");
        launch_quantize_acts(x, n, a->qx, a->xs, a->xsum, s);
    }
    hipError_t e = hipMemcpyAsync(qw, a->qx, (size_t)n, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(sw, a->xs, (size_t)(n / 32) * 4, hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return latch(b, hip_fail(a->d, e, "quantize"));
    return launched(b, "quantize");
}

// internal/gpu/batch.go:271-275 QuantizeFP8: E4M3 codes and block scales
// into the products' scratch, and, as the reference leaves them in the
// arena (internal/gpu/mx.go:146-172), the codes' values, unscaled, as n
// float32 words at qx_off and the block scales at xs_off. (A NaN code, from
// an input block holding an infinity or NaN, reads as NaN, the CPU path's
// value in num.ActFP8.Vals; the reference's Vulkan kernel gives ±480 there.)
int rk_batch_quantize_fp8(rk_batch *b, int64_t in, int64_t n) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    rk_arena *a = b->a;
    if (a->qx_off < 0) return latch(b, fail(a->d, RK_ERR_ARGS, "gpu: arena has no scratch for quantized inputs"));
    if (n % 32 != 0 || n > kMaxCols) return latch(b, fail(a->d, RK_ERR_ARGS, "gpu: quantize of %lld floats", (long long)n));
    const float *x = span(b, in, n, "quantize input");
    float *vw = x ? span(b, a->qx_off, n, "quantized values") : nullptr;
    float *sw = vw ? span(b, a->xs_off, n / 32, "quantized scales") : nullptr;
    if (!sw) return b->err;
    hipStream_t s = a->d->stream;
    {
        ProfScope p(a->d, s, "act_fp8");
        launch_act_fp8(x, n, reinterpret_cast<uint8_t *>(a->qx), a->xs, s);
    }
    {
        ProfScope p(a->d, s, "e4m3_values");
        launch_e4m3_values(reinterpret_cast<const uint8_t *>(a->qx), n, vw, s);
    }
    hipError_t e = hipMemcpyAsync(sw, a->xs, (size_t)(n / 32) * 4, hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return latch(b, hip_fail(a->d, e, "quantize"));
    return launched(b, "quantize");
}

// internal/gpu/dsbatch.go:142-172 ExpertMatVecs: the inputs quantized into
// the arena's quantize scratch (input k at k·cols codes), then one launch
// over the slots.
int rk_batch_expert_matvecs(rk_batch *b, rk_matrix *m, int64_t per_expert, int64_t ids, int32_t slots, int64_t in,
                            int64_t in_stride, int32_t div, int64_t out, int64_t out_stride) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    rk_arena *a = b->a;
    rk_device *d = a->d;
    if (!m || m->d != d || m->kind != RK_FP4 || per_expert <= 0 || m->rows % per_expert != 0)
        return latch(b, fail(d, RK_ERR_ARGS, "gpu: not a matrix of E2M1 experts"));
    if (per_expert % 8 != 0)
        return latch(b, fail(d, RK_ERR_UNSUPPORTED, "gpu: experts of %lld rows (this build takes multiples of 8)",
                             (long long)per_expert));
    if (slots <= 0) return RK_OK;
    if (div < 0) return latch(b, fail(d, RK_ERR_ARGS, "rk_batch_expert_matvecs: negative div"));
    if (div == 0) div = slots;
    if (a->qx_off < 0) return latch(b, fail(d, RK_ERR_ARGS, "gpu: arena has no scratch for quantized inputs"));
    const int64_t cols = m->cols, inputs = (slots + div - 1) / div;
    if (inputs * cols > kMaxCols)
        return latch(b, fail(d, RK_ERR_ARGS, "gpu: %lld inputs of %lld floats exceed the quantize scratch",
                             (long long)inputs, (long long)cols));
    const float *idw = span(b, ids, slots, "expert ids");
    if (!idw) return b->err;
    for (int32_t k = 0; k < slots; k++)
        if (!span(b, out + k * out_stride, per_expert, "expert output")) return b->err;
    float *o = a->buf + out;
    hipStream_t s = d->stream;
    {
        ProfScope p(d, s, "act_fp8");
        for (int64_t k = 0; k < inputs; k++) {
            const float *x = span(b, in + k * in_stride, cols, "expert input");
            if (!x) return b->err;
            launch_act_fp8(x, cols, reinterpret_cast<uint8_t *>(a->qx) + k * cols, a->xs + k * (cols / 32), s);
        }
    }
    ProfScope p(d, s, "matvec_fp4_experts");
    launch_mx_experts(m->w, m->e8m0, m->rows / per_expert, per_expert, cols, reinterpret_cast<const uint32_t *>(idw),
                      slots, div, reinterpret_cast<const uint8_t *>(a->qx), a->xs, o, out_stride, m->raw != 0, s);
    return launched(b, "expert products");
}

// internal/gpu/dsbatch.go:174-210 MatVecsBatch: m times n inputs, one
// product an input (each input quantized once). A kernel reading an E4M3
// matrix once for several inputs measured slower on MI355X than the
// products one by one (its float64 block sums per input make it
// compute-bound: 14.5 µs an input against about 10 µs a product at
// 5120x8192), so the weights are read once an input.
int rk_batch_matvecs_batch(rk_batch *b, rk_matrix *m, int64_t out, int64_t out_stride, int64_t in, int64_t in_stride,
                           int32_t n) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    if (!m || m->d != b->a->d) return latch(b, fail(b->a->d, RK_ERR_ARGS, "gpu: matrix on another device"));
    for (int32_t j = 0; j < n; j++) {
        const int64_t o = out + j * out_stride;
        int rc = rk_batch_matvecs(b, 1, &m, &o, in + j * in_stride);
        if (rc) return rc;
    }
    return RK_OK;
}

// internal/gpu/dsbatch.go:60-74 ActQuantInPlace and FP4QuantInPlace.
int rk_batch_act_quant_inplace(rk_batch *b, int64_t off, int64_t n) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    if (n < 0 || n % 32 != 0) return latch(b, fail(b->a->d, RK_ERR_ARGS, "gpu: act quant of %lld floats", (long long)n));
    float *x = span(b, off, n, "act quant");
    if (!x) return b->err;
    ProfScope p(b->a->d, b->a->d->stream, "act_quant_inplace");
    launch_act_quant_inplace(x, n, b->a->d->stream);
    return launched(b, "act quant");
}

int rk_batch_fp4_quant_inplace(rk_batch *b, int64_t off, int64_t n, int32_t e4m3) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    if (n < 0 || n % (e4m3 ? 16 : 32) != 0)
        return latch(b, fail(b->a->d, RK_ERR_ARGS, "gpu: fp4 quant of %lld floats", (long long)n));
    float *x = span(b, off, n, "fp4 quant");
    if (!x) return b->err;
    ProfScope p(b->a->d, b->a->d->stream, "fp4_quant_inplace");
    launch_fp4_quant_inplace(x, n, e4m3 != 0, b->a->d->stream);
    return launched(b, "fp4 quant");
}

// internal/gpu/batch.go:282-287 RMSNorm.
int rk_batch_rmsnorm(rk_batch *b, rk_vectors *vecs, int64_t in, int64_t out, int64_t w, int32_t n, int32_t segs,
                     int64_t stride, float recip_n, float eps) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    if (n <= 0 || segs <= 0 || (segs > 1 && stride < 0))
        return latch(b, fail(b->a->d, RK_ERR_ARGS, "rk_batch_rmsnorm: bad shape"));
    const int64_t extent = (int64_t)(segs - 1) * stride + n;
    float *xi = span(b, in, extent, "rmsnorm input");
    float *xo = xi ? span(b, out, extent, "rmsnorm output") : nullptr;
    const float *wv = xo ? vspan(b, vecs, w, n, "rmsnorm weights") : nullptr;
    if (!wv) return b->err;
    ProfScope p(b->a->d, b->a->d->stream, "rmsnorm");
    launch_rmsnorm(xi, xo, wv, n, segs, stride, recip_n, eps, b->a->d->stream);
    return launched(b, "rmsnorm");
}

// internal/gpu/batch.go:289-292 AddVec.
int rk_batch_addvec(rk_batch *b, rk_vectors *vecs, int64_t out, int64_t v, int64_t n) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    float *o = span(b, out, n, "addvec output");
    const float *vv = o ? vspan(b, vecs, v, n, "addvec vector") : nullptr;
    if (!vv) return b->err;
    ProfScope p(b->a->d, b->a->d->stream, "addvec");
    launch_addvec(o, vv, n, b->a->d->stream);
    return launched(b, "addvec");
}

// internal/gpu/batch.go:294-298 Rope.
int rk_batch_rope(rk_batch *b, int64_t q, int64_t k, int32_t q_dim, int32_t kv_dim, int32_t head_size, int64_t cos,
                  int64_t sin) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    if (head_size <= 0 || head_size % 2 || q_dim % 2 || kv_dim < 0 || kv_dim > q_dim)
        return latch(b, fail(b->a->d, RK_ERR_ARGS, "rk_batch_rope: bad shape"));
    float *qq = span(b, q, q_dim, "rope q");
    float *kk = qq ? span(b, k, kv_dim, "rope k") : nullptr;
    const float *c = kk ? span(b, cos, head_size / 2, "rope cos") : nullptr;
    const float *sn = c ? span(b, sin, head_size / 2, "rope sin") : nullptr;
    if (!sn) return b->err;
    ProfScope p(b->a->d, b->a->d->stream, "rope");
    launch_rope(qq, kk, q_dim, kv_dim, head_size, c, sn, b->a->d->stream);
    return launched(b, "rope");
}

// internal/gpu/batch.go:300-303 Copy.
int rk_batch_copy(rk_batch *b, int64_t src, int64_t dst, int64_t n) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    const float *s = span(b, src, n, "copy source");
    float *t = s ? span(b, dst, n, "copy destination") : nullptr;
    if (!t) return b->err;
    ProfScope p(b->a->d, b->a->d->stream, "copy");
    launch_copy(s, t, n, b->a->d->stream);
    return launched(b, "copy");
}

// internal/gpu/batch.go:305-316 Attention.
int rk_batch_attention(rk_batch *b, int64_t q, int64_t keys, int64_t vals, int64_t att, int64_t att_stride, int64_t out,
                       int32_t positions, int32_t heads, int32_t kv_heads, int32_t head_size, int32_t kv_dim,
                       float inv_sqrt) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    if (positions <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads || head_size <= 0 ||
        (int64_t)kv_heads * head_size > kv_dim || att_stride < positions)
        return latch(b, fail(b->a->d, RK_ERR_ARGS, "rk_batch_attention: bad shape"));
    const int64_t qd = (int64_t)heads * head_size, cache = (int64_t)positions * kv_dim;
    const float *qq = span(b, q, qd, "attention q");
    const float *kk = qq ? span(b, keys, cache, "attention keys") : nullptr;
    const float *vv = kk ? span(b, vals, cache, "attention values") : nullptr;
    float *aa = vv ? span(b, att, (int64_t)(heads - 1) * att_stride + positions, "attention scores") : nullptr;
    float *oo = aa ? span(b, out, qd, "attention output") : nullptr;
    if (!oo) return b->err;
    ProfScope p(b->a->d, b->a->d->stream, "attention");
    launch_attention(qq, kk, vv, aa, att_stride, oo, positions, heads, kv_heads, head_size, kv_dim, inv_sqrt,
                     b->a->d->stream);
    return launched(b, "attention");
}

// internal/gpu/batch.go:318-326 Residual.
int rk_batch_residual(rk_batch *b, int64_t x, int64_t y, int64_t n, int32_t canonical) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    float *xx = span(b, x, n, "residual x");
    const float *yy = xx ? span(b, y, n, "residual y") : nullptr;
    if (!yy) return b->err;
    ProfScope p(b->a->d, b->a->d->stream, "residual");
    launch_residual(xx, yy, n, canonical != 0, b->a->d->stream);
    return launched(b, "residual");
}

// internal/gpu/batch.go:328-331 SiluMul.
int rk_batch_silumul(rk_batch *b, int64_t a_off, int64_t b_off, int64_t n) {
    if (!b) return RK_ERR_ARGS;
    if (b->err) return b->err;
    float *aa = span(b, a_off, n, "silumul a");
    const float *bb = aa ? span(b, b_off, n, "silumul b") : nullptr;
    if (!bb) return b->err;
    ProfScope p(b->a->d, b->a->d->stream, "silumul");
    launch_silumul(aa, bb, n, b->a->d->stream);
    return launched(b, "silumul");
}

// internal/gpu/batch.go:333-349 Submit: run, wait, deliver reads, release.
int rk_batch_submit(rk_batch *b) {
    if (!b) return RK_ERR_ARGS;
    rk_arena *a = b->a;
    rk_device *d = a->d;
    int rc = b->err;
    hipError_t e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        if (rc == RK_OK) rc = hip_fail(d, e, "submit");
    }
    if (rc == RK_OK)
        for (auto &r : b->reads) memcpy(r.dst, a->staging + r.at, (size_t)r.n * 4);
    delete b;
    d->gate.release();
    return rc;
}

}  // extern "C"
