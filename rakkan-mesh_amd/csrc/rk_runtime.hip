// rk_runtime.hip — host side of librkhip: devices, matrices and the C-ABI
// entry points of include/rk.h for them. The object model mirrors
// internal/gpu (Device, Matrix, MulVecs); each C entry point cites the Go
// function whose body it replaces.
#include "rk_mm.h"
#include "rk_runtime.h"

#include "rk_dense.h"
#include "rk_mx.h"
#include "rk_fused.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <vector>

namespace rk {

thread_local std::string g_open_error;
thread_local LaunchEvents *g_launch_events = nullptr;

int fail(rk_device *d, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (d)
        d->err = buf;
    else
        g_open_error = buf;
    return code;
}

int hip_fail(rk_device *d, hipError_t e, const char *what) {
    return fail(d, e == hipErrorOutOfMemory ? RK_ERR_OOM : RK_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int dev_alloc(rk_device *d, void **p, size_t bytes, const char *what) {
    hipError_t e = hipMalloc(p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        return hip_fail(d, e, what);
    }
    return RK_OK;
}

// Serialise use of the device's shared scratch across streams: stream order
// already serialises uses from one stream; when a call comes on another
// stream, an event recorded on the previous one (marking all work enqueued
// there so far) is waited for first.
int scratch_acquire(rk_device *d, hipStream_t s) {
    if (d->capturing) return RK_OK;  // a recorded graph runs on one stream
    if (d->scratch_stream_set && d->scratch_stream != s) {
        HIP_TRY(d, hipEventRecord(d->scratch_free, d->scratch_stream), "scratch record");
        HIP_TRY(d, hipStreamWaitEvent(s, d->scratch_free, 0), "scratch wait");
    }
    d->scratch_stream = s;
    d->scratch_stream_set = true;
    return RK_OK;
}

static hipEvent_t take_event(rk_device *d) {
    if (!d->event_pool.empty()) {
        hipEvent_t e = d->event_pool.back();
        d->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return e;
}

ProfScope::ProfScope(rk_device *d, hipStream_t, const char *kernel) {
    if (!d->profiling || d->capturing) return;
    hipEvent_t a = take_event(d), b = take_event(d);
    if (!a || !b) {
        if (a) d->event_pool.push_back(a);
        if (b) d->event_pool.push_back(b);
        return;
    }
    d_ = d;
    kernel_ = kernel;
    ev_ = LaunchEvents{a, b, false};
    g_launch_events = &ev_;
}

ProfScope::~ProfScope() {
    g_launch_events = nullptr;
    if (!d_) return;
    if (ev_.launched) {
        d_->prof.push_back({kernel_, ev_.start, ev_.stop});
    } else {  // never recorded: back to the pool
        d_->event_pool.push_back(ev_.start);
        d_->event_pool.push_back(ev_.stop);
    }
}

// Device bytes held (Device.Used), under the accounting lock.
void add_used(rk_device *d, int64_t bytes) {
    std::lock_guard<std::mutex> g(d->mu);
    d->used += bytes;
}

// Products of n matrices sharing cols with one input: each run of up to
// three matrices of one format is one launch. Inputs up to 8192 wide that
// are 16-byte aligned are quantized by every workgroup into LDS (no extra
// launch; measured faster there); wider or unaligned ones by one quantize
// launch into the scratch q, which the products then read.
int enqueue_matvecs(rk_device *d, int32_t n, rk_matrix *const *ms, float *const *outs, const float *x, int64_t cols,
                    const QScratch &q, hipStream_t s) {
    const bool aligned = ((uintptr_t)x & 15) == 0;
    const bool in_lds = cols <= 8192 && aligned && fused_fits(kProQuant, (int)cols);
    bool quantized = false;
    for (int kind : {RK_Q8, RK_Q4}) {
        FusedArgs a{};
        a.cols = (int32_t)cols;
        // each workgroup quantizes x itself, unless the input is wide and no
        // static-schedule instance takes it (then one quantize launch first)
        const bool q_in = in_lds || (aligned && cols <= kMaxLdsCols &&
                                     stream_has(kind == RK_Q8 ? kFmtQ8 : kFmtQ4, kProQuant, kEpStore, (int)cols));
        auto flush = [&]() -> int {
            if (a.nseg == 0) return RK_OK;
            int pro = kProQuant;
            if (q_in) {
                a.x = x;
            } else {
                if (!quantized) {
                    ProfScope p(d, s, "quantize_acts");
                    launch_quantize_acts(x, cols, q.qx, q.xs, q.xsum, s);
                    quantized = true;
                }
                pro = kProGlobal;
                a.qx = q.qx;
                a.xs = q.xs;
                a.xsum = q.xsum;
            }
            bool ok;
            {
                ProfScope p(d, s, kind == RK_Q8 ? "matvec_q8" : "matvec_q4");
                ok = launch_fused(kind == RK_Q8 ? kFmtQ8 : kFmtQ4, pro, kEpStore, a, d->cu, s);
            }
            a.nseg = 0;
            a.rows = 0;
            return ok ? RK_OK : fail(d, RK_ERR_UNSUPPORTED, "matvec: width %lld has no kernel", (long long)cols);
        };
        for (int i = 0; i < n; i++) {
            if (ms[i]->kind != kind) continue;
            a.seg[a.nseg] = MatSeg{ms[i]->w, ms[i]->scales, outs[i], ms[i]->rows};
            a.rows += (int32_t)ms[i]->rows;
            if (++a.nseg == 3) {
                int rc = flush();
                if (rc) return rc;
            }
        }
        int rc = flush();
        if (rc) return rc;
    }
    // E4M3 / E2M1 matrices: the input quantized once to E4M3 with block
    // scales into the scratch (internal/gpu/batch.go:221-233 QuantizeFP8),
    // then one launch each. (Quantizing inside the products was measured
    // slower: every workgroup of a few rows quantizes the whole input.)
    bool mx_quantized = false;
    for (int i = 0; i < n; i++) {
        if (ms[i]->kind != RK_FP8 && ms[i]->kind != RK_FP4) continue;
        if (!mx_quantized) {
            ProfScope p(d, s, "act_fp8");
            launch_act_fp8(x, cols, reinterpret_cast<uint8_t *>(q.qx), q.xs, s);
            mx_quantized = true;
        }
        ProfScope p(d, s, ms[i]->kind == RK_FP8 ? "matvec_fp8" : "matvec_fp4");
        launch_mx_matvec(ms[i]->kind == RK_FP4, ms[i]->w, ms[i]->e8m0, ms[i]->rows, cols,
                         reinterpret_cast<const uint8_t *>(q.qx), q.xs, outs[i], ms[i]->raw != 0, s);
    }
    // float32 / bfloat16 matrices take x as it is (internal/gpu/batch.go:
    // 263-264: no quantized input), one launch each
    for (int i = 0; i < n; i++) {
        if (ms[i]->kind != RK_F32 && ms[i]->kind != RK_BF16) continue;
        ProfScope p(d, s, ms[i]->kind == RK_BF16 ? "matvec_bf16" : "matvec_f32");
        launch_dense_matvec(ms[i]->kind == RK_BF16, ms[i]->w, ms[i]->rows, cols, x, outs[i], s);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(d, e, "matvec launch");
    return RK_OK;
}

// internal/gpu/batch.go:221-238: one input is quantized either to Q8_0 or
// to E4M3, not both.
int mixed_inputs(rk_device *d, int32_t n, rk_matrix *const *ms) {
    bool q8 = false, fp8 = false;
    for (int i = 0; i < n; i++) {
        q8 = q8 || ms[i]->kind == RK_Q8 || ms[i]->kind == RK_Q4;
        fp8 = fp8 || ms[i]->kind == RK_FP8 || ms[i]->kind == RK_FP4;
    }
    return q8 && fp8 ? fail(d, RK_ERR_ARGS, "gpu: Q8_0 and FP8 products of one input") : RK_OK;
}

int check_products(rk_device *d, int32_t n, rk_matrix *const *ms, int64_t cols, int64_t *total) {
    if (!d || n < 0 || (n > 0 && !ms)) return fail(d, RK_ERR_ARGS, "rk_matvecs: bad arguments");
    *total = 0;
    for (int i = 0; i < n; i++) {
        rk_matrix *m = ms[i];
        if (!m || m->d != d) return fail(d, RK_ERR_ARGS, "rk_matvecs: matrix %d is on another device", i);
        if (m->cols != cols)
            return fail(d, RK_ERR_ARGS, "gpu: %lld×%lld matrix times %lld", (long long)m->rows, (long long)m->cols,
                        (long long)cols);
        if (m->kind < RK_F32 || m->kind > RK_FP4)
            return fail(d, RK_ERR_UNSUPPORTED, "rk_matvecs: format %d has no kernel in this build", m->kind);
        *total += m->rows;
    }
    return mixed_inputs(d, n, ms);
}

// Grows a device buffer to `need` elements of `elem` bytes (contents not
// kept). Work already enqueued on any stream may still use the old buffer,
// so the device is drained first.
static int grow(rk_device *d, void **p, int64_t &cap, int64_t need, size_t elem, const char *what) {
    if (need <= cap) return RK_OK;
    if (d->capturing) return fail(d, RK_ERR_ARGS, "%s: scratch must grow, which cannot be recorded", what);
    HIP_TRY(d, hipDeviceSynchronize(), what);
    (void)hipFree(*p);
    *p = nullptr;
    cap = 0;
    int rc = dev_alloc(d, p, (size_t)need * elem, what);
    if (rc) return rc;
    cap = need;
    return RK_OK;
}

// The batched products' quantized input for `codes` codes (tokens·cols).
static int batch_scratch(rk_device *d, int64_t codes) {
    if (codes <= d->bq_cap) return RK_OK;
    if (d->capturing) return fail(d, RK_ERR_ARGS, "batch scratch must grow, which cannot be recorded");
    HIP_TRY(d, hipDeviceSynchronize(), "batch scratch");
    (void)hipFree(d->bqx);
    (void)hipFree(d->bxs);
    (void)hipFree(d->bxsum);
    d->bqx = nullptr;
    d->bxs = nullptr;
    d->bxsum = nullptr;
    d->bq_cap = 0;
    int rc;
    if ((rc = dev_alloc(d, (void **)&d->bqx, (size_t)codes, "batch scratch")) ||
        (rc = dev_alloc(d, (void **)&d->bxs, (size_t)(codes / 32) * 4, "batch scratch")) ||
        (rc = dev_alloc(d, (void **)&d->bxsum, (size_t)(codes / 32) * 4, "batch scratch")))
        return rc;
    d->bq_cap = codes;
    return RK_OK;
}

// Batched products: quantize the tokens' inputs once, then one MFMA launch
// per format (up to three matrices each).
int enqueue_matmuls(rk_device *d, int32_t n, rk_matrix *const *ms, float *const *outs, const float *x, int64_t cols,
                    int32_t tokens, const QScratch &q, hipStream_t s) {
    {
        ProfScope p(d, s, "quantize_acts");
        launch_quantize_acts(x, cols * tokens, q.qx, q.xs, q.xsum, s);
    }
    for (int kind : {RK_Q8, RK_Q4}) {
        MmArgs a{};
        a.cols = (int32_t)cols;
        a.tokens = tokens;
        a.qx = q.qx;
        a.xs = q.xs;
        auto flush = [&]() -> int {
            if (a.nseg == 0) return RK_OK;
            bool ok;
            {
                ProfScope p(d, s, kind == RK_Q8 ? "matmul_q8" : "matmul_q4");
                ok = launch_mm(kind == RK_Q8 ? kFmtQ8 : kFmtQ4, kEpStore, a, s);
            }
            a.nseg = 0;
            a.rows = 0;
            return ok ? RK_OK : fail(d, RK_ERR_UNSUPPORTED, "matmul: shape has no kernel");
        };
        for (int i = 0; i < n; i++) {
            if (ms[i]->kind != kind) continue;
            a.seg[a.nseg] = MatSeg{ms[i]->w, ms[i]->scales, outs[i], ms[i]->rows};
            a.rows += (int32_t)ms[i]->rows;
            if (++a.nseg == 3) {
                int rc = flush();
                if (rc) return rc;
            }
        }
        int rc = flush();
        if (rc) return rc;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(d, e, "matmul launch");
    return RK_OK;
}

int check_matmul(rk_device *d, int32_t n, rk_matrix *const *ms, int64_t cols, int32_t tokens, int64_t *total) {
    int rc = check_products(d, n, ms, cols, total);
    if (rc) return rc;
    for (int i = 0; i < n; i++)
        if (ms[i]->kind != RK_Q8 && ms[i]->kind != RK_Q4)
            return fail(d, RK_ERR_UNSUPPORTED, "rk_matmul_t: format %d has no batched kernel in this build",
                        ms[i]->kind);
    if (tokens < 0) return fail(d, RK_ERR_ARGS, "rk_matmul_t: %d tokens", tokens);
    if ((int64_t)tokens * cols > ((int64_t)1 << 31) - 32 || (int64_t)tokens * *total > ((int64_t)1 << 31))
        return fail(d, RK_ERR_ARGS, "rk_matmul_t: %d tokens of %lld columns is too large for one call", tokens,
                    (long long)cols);
    return RK_OK;
}

// internal/gpu/device.go:587-597, 619-621 Upload of float32 / bfloat16
// rows (bfloat16 rows need an even width). Each row is stored padded with
// zeros to dense_row_elems(cols) elements (the products' layout).
static int upload_dense(rk_device *d, int32_t kind, int64_t rows, int64_t cols, const void *w, rk_matrix **out) {
    if (kind == RK_BF16 && cols % 2 != 0) return fail(d, RK_ERR_ARGS, "gpu: bfloat16 rows need an even width");
    const size_t es = kind == RK_BF16 ? 2 : 4;
    const int64_t pitch = dense_row_elems(cols) * (int64_t)es;
    const int64_t wbytes = rows * pitch;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    rk_matrix *m = new rk_matrix();
    m->d = d;
    m->kind = kind;
    m->rows = rows;
    m->cols = cols;
    int rc = dev_alloc(d, (void **)&m->w, (size_t)wbytes, "matrix");
    if (rc) {
        delete m;
        return rc;
    }
    hipError_t e = hipMemsetAsync(m->w, 0, (size_t)wbytes, d->stream);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(m->w, (size_t)pitch, w, (size_t)cols * es, (size_t)cols * es, (size_t)rows,
                             hipMemcpyHostToDevice, d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) {
        (void)hipFree(m->w);
        delete m;
        return hip_fail(d, e, "matrix upload");
    }
    m->bytes = wbytes;
    add_used(d, m->bytes);
    *out = m;
    return RK_OK;
}

}  // namespace rk

using namespace rk;

extern "C" {

int rk_device_count(int32_t *count) {
    if (!count) return RK_ERR_ARGS;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *count = 0;
        return RK_OK;  // no runtime devices: an empty list, as Devices()
    }
    *count = n;
    return RK_OK;
}

int rk_device_info_get(int32_t index, rk_device_info *info) {
    if (!info) return RK_ERR_ARGS;
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, index);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(nullptr, RK_ERR_NO_DEVICE, "device %d: %s", index, hipGetErrorString(e));
    }
    memset(info, 0, sizeof *info);
    info->index = index;
    snprintf(info->name, sizeof info->name, "%s", p.name);
    snprintf(info->arch, sizeof info->arch, "%s", p.gcnArchName);
    info->memory = (int64_t)p.totalGlobalMem;
    info->compute_units = p.multiProcessorCount;
    // The kernels are built for gfx950 with f32 denormals kept and
    // round-to-nearest-even: exact there, and nowhere else.
    info->exact = strncmp(p.gcnArchName, "gfx950", 6) == 0;
    info->integrated = p.integrated != 0;
    return RK_OK;
}

int rk_device_open(int32_t index, rk_device **out) {
    if (!out) return RK_ERR_ARGS;
    *out = nullptr;
    rk_device_info info;
    int rc = rk_device_info_get(index, &info);
    if (rc != RK_OK) return rc;
    if (!info.exact)
        return fail(nullptr, RK_ERR_NO_DEVICE, "device %d is %s; this build runs on gfx950 only", index, info.arch);
    hipError_t e = hipSetDevice(index);
    if (e != hipSuccess) return hip_fail(nullptr, e, "hipSetDevice");
    rk_device *d = new rk_device();
    d->index = index;
    d->cu = info.compute_units;
    d->info = info;
    auto bail = [&](int code) {
        if (!d->err.empty()) g_open_error = d->err;
        rk_device_close(d);
        return code;
    };
    if ((e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking)) != hipSuccess)
        return bail(hip_fail(d, e, "stream"));
    if ((e = hipEventCreateWithFlags(&d->scratch_free, hipEventDisableTiming)) != hipSuccess)
        return bail(hip_fail(d, e, "event"));
    if ((rc = dev_alloc(d, (void **)&d->x, 4 * kMaxCols, "scratch")) ||
        (rc = dev_alloc(d, (void **)&d->qx, kMaxCols, "scratch")) ||
        (rc = dev_alloc(d, (void **)&d->xs, 4 * (kMaxCols / 32), "scratch")) ||
        (rc = dev_alloc(d, (void **)&d->xsum, 4 * (kMaxCols / 32), "scratch")) ||
        (rc = dev_alloc(d, (void **)&d->out, 4 * kMaxRows, "scratch")))
        return bail(rc);
    if ((e = hipHostMalloc((void **)&d->h_stage, 4 * (kMaxCols + kMaxRows), hipHostMallocDefault)) != hipSuccess)
        return bail(hip_fail(d, e, "pinned staging"));
    if ((rc = noalloc_setup(d))) return bail(rc);
    *out = d;
    return RK_OK;
}

int rk_device_close(rk_device *d) {
    if (!d) return RK_ERR_ARGS;
    (void)hipSetDevice(d->index);
    if (d->stream) (void)hipStreamSynchronize(d->stream);
    (void)hipFree(d->x);
    (void)hipFree(d->qx);
    (void)hipFree(d->xs);
    (void)hipFree(d->xsum);
    (void)hipFree(d->out);
    (void)hipFree(d->bqx);
    (void)hipFree(d->bxs);
    (void)hipFree(d->bxsum);
    (void)hipFree(d->bx);
    (void)hipFree(d->bout);
    if (d->h_stage) (void)hipHostFree(d->h_stage);
    if (d->scratch_free) (void)hipEventDestroy(d->scratch_free);
    for (auto &r : d->prof) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    for (hipEvent_t e : d->event_pool) (void)hipEventDestroy(e);
    if (d->stream) (void)hipStreamDestroy(d->stream);
    (void)hipGetLastError();
    delete d;
    return RK_OK;
}

int64_t rk_used_bytes(rk_device *d) {
    if (!d) return -1;
    std::lock_guard<std::mutex> g(d->mu);
    return d->used;  // read under the accounting lock only
}

const char *rk_last_error(rk_device *d) { return d ? d->err.c_str() : g_open_error.c_str(); }

int rk_matrix_upload(rk_device *d, int32_t kind, int64_t rows, int64_t cols, const void *w, const float *scales,
                     rk_matrix **out) {
    if (!d || !out || !w) return fail(d, RK_ERR_ARGS, "rk_matrix_upload: null argument");
    *out = nullptr;
    // internal/gpu/device.go:619-624 shape checks.
    if (rows <= 0 || cols <= 0 || cols > kMaxCols || rows > (int64_t)1 << 24)
        return fail(d, RK_ERR_ARGS, "gpu: matrix %lld×%lld out of range", (long long)rows, (long long)cols);
    int64_t wbytes = 0;
    switch (kind) {
    case RK_Q8: wbytes = rows * cols; break;
    case RK_Q4: wbytes = rows * cols / 2; break;
    case RK_F32:
    case RK_BF16: return upload_dense(d, kind, rows, cols, w, out);
    case RK_FP8:
    case RK_FP4: return fail(d, RK_ERR_ARGS, "rk_matrix_upload: E4M3 / E2M1 matrices go through rk_matrix_upload_mx");
    default: return fail(d, RK_ERR_ARGS, "rk_matrix_upload: unknown format %d", kind);
    }
    if (cols % 32 != 0 || !scales) return fail(d, RK_ERR_ARGS, "gpu: quantized matrix of the wrong shape");
    const int64_t sbytes = rows * (cols / 32) * 4;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    rk_matrix *m = new rk_matrix();
    m->d = d;
    m->kind = kind;
    m->rows = rows;
    m->cols = cols;
    int rc;
    if ((rc = dev_alloc(d, (void **)&m->w, (size_t)wbytes, "matrix")) ||
        (rc = dev_alloc(d, (void **)&m->scales, (size_t)sbytes, "matrix scales"))) {
        (void)hipFree(m->w);
        delete m;
        return rc;
    }
    hipError_t e = hipMemcpyAsync(m->w, w, (size_t)wbytes, hipMemcpyHostToDevice, d->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(m->scales, scales, (size_t)sbytes, hipMemcpyHostToDevice, d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) {
        (void)hipFree(m->w);
        (void)hipFree(m->scales);
        delete m;
        return hip_fail(d, e, "matrix upload");
    }
    m->bytes = wbytes + sbytes;
    add_used(d, m->bytes);
    *out = m;
    return RK_OK;
}

// internal/gpu/device.go:587-700 Upload of Format{FP8 | FP4, E8M0}: codes
// [rows][row bytes] and their scale bytes as given.
int rk_matrix_upload_mx_chunks(rk_device *d, int32_t kind, int64_t rows, int64_t cols, int32_t n_w,
                               const uint8_t *const *w, const int64_t *w_len, int32_t n_s,
                               const uint8_t *const *e8m0, const int64_t *s_len, int32_t align_rows,
                               rk_matrix **out) {
    if (!d || !out || n_w <= 0 || n_s <= 0 || !w || !w_len || !e8m0 || !s_len)
        return fail(d, RK_ERR_ARGS, "rk_matrix_upload_mx: null argument");
    *out = nullptr;
    if (kind != RK_FP8 && kind != RK_FP4) return fail(d, RK_ERR_ARGS, "rk_matrix_upload_mx: format %d", kind);
    // the pieces, each read as one run of bytes (device.go:704-723 gatherer)
    int64_t wtot = 0, stot = 0;
    for (int32_t i = 0; i < n_w; i++) {
        if (w_len[i] < 0 || (w_len[i] > 0 && !w[i])) return fail(d, RK_ERR_ARGS, "rk_matrix_upload_mx: null chunk");
        wtot += w_len[i];
    }
    for (int32_t i = 0; i < n_s; i++) {
        if (s_len[i] < 0 || (s_len[i] > 0 && !e8m0[i]))
            return fail(d, RK_ERR_ARGS, "rk_matrix_upload_mx: null chunk");
        stot += s_len[i];
    }
    const int64_t row_bytes = kind == RK_FP8 ? cols : cols / 2;
    if (rows <= 0 || cols <= 0 || cols > kMaxCols || rows > (int64_t)1 << 24 || wtot != rows * row_bytes)
        return fail(d, RK_ERR_ARGS, "gpu: matrix %lld×%lld out of range", (long long)rows, (long long)cols);
    const int64_t nb = cols / 32;
    const int64_t blocks = kind == RK_FP8 ? (rows + 31) / 32 * nb : rows * nb;
    if (cols % 32 != 0 || stot != blocks) return fail(d, RK_ERR_ARGS, "gpu: block-scaled matrix of the wrong shape");
    if (kind == RK_FP8) {  // num.ValidE4M3: the NaN codes are refused
        for (int32_t c = 0; c < n_w; c++)
            for (int64_t i = 0; i < w_len[c]; i++)
                if ((w[c][i] & 0x7f) == 0x7f) return fail(d, RK_ERR_ARGS, "gpu: NaN in E4M3 weights");
    }
    // device.go:611-618: runs of align_rows rows (an expert's) kept whole.
    // One allocation holds every row here, so the runs are whole already;
    // the shape rule is the reference's.
    if (align_rows > 0 && (rows % align_rows != 0 || (kind == RK_FP8 && align_rows % 32 != 0)))
        return fail(d, RK_ERR_ARGS, "gpu: rows not a whole number of aligned runs");
    // the scale bytes (small) gathered on the host; E2M1's repacked into the
    // products' tile layout
    std::vector<uint8_t> sc((size_t)blocks);
    {
        int64_t at = 0;
        for (int32_t c = 0; c < n_s; c++) {
            if (s_len[c]) memcpy(sc.data() + at, e8m0[c], (size_t)s_len[c]);
            at += s_len[c];
        }
    }
    const int64_t sbytes = kind == RK_FP8 ? blocks : mx_fp4_scale_bytes(rows, cols);
    std::vector<uint8_t> packed;
    const uint8_t *sdev = sc.data();
    if (kind == RK_FP4) {
        packed.resize((size_t)sbytes);
        mx_fp4_pack_scales(sc.data(), rows, cols, packed.data());
        sdev = packed.data();
    }
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    rk_matrix *m = new rk_matrix();
    m->d = d;
    m->kind = kind;
    m->rows = rows;
    m->cols = cols;
    int rc;
    if ((rc = dev_alloc(d, (void **)&m->w, (size_t)wtot, "matrix")) ||
        (rc = dev_alloc(d, (void **)&m->e8m0, (size_t)sbytes, "matrix scales"))) {
        (void)hipFree(m->w);
        delete m;
        return rc;
    }
    // the codes piece by piece into place: never gathered on the host
    hipError_t e = hipSuccess;
    int64_t at = 0;
    for (int32_t c = 0; c < n_w && e == hipSuccess; c++) {
        if (w_len[c]) e = hipMemcpyAsync(m->w + at, w[c], (size_t)w_len[c], hipMemcpyHostToDevice, d->stream);
        at += w_len[c];
    }
    if (e == hipSuccess) e = hipMemcpyAsync(m->e8m0, sdev, (size_t)sbytes, hipMemcpyHostToDevice, d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(m->w);
        (void)hipFree(m->e8m0);
        delete m;
        return hip_fail(d, e, "matrix upload");
    }
    m->bytes = wtot + sbytes;
    add_used(d, m->bytes);
    *out = m;
    return RK_OK;
}

int rk_matrix_upload_mx(rk_device *d, int32_t kind, int64_t rows, int64_t cols, const uint8_t *w,
                        const uint8_t *e8m0, rk_matrix **out) {
    if (!d || !out || !w || !e8m0) return fail(d, RK_ERR_ARGS, "rk_matrix_upload_mx: null argument");
    if (rows <= 0 || cols <= 0 || cols > kMaxCols || rows > (int64_t)1 << 24) {
        *out = nullptr;
        return fail(d, RK_ERR_ARGS, "gpu: matrix %lld×%lld out of range", (long long)rows, (long long)cols);
    }
    const int64_t wlen = kind == RK_FP8 ? rows * cols : rows * (cols / 2);
    const int64_t slen = kind == RK_FP8 ? (rows + 31) / 32 * (cols / 32) : rows * (cols / 32);
    return rk_matrix_upload_mx_chunks(d, kind, rows, cols, 1, &w, &wlen, 1, &e8m0, &slen, 0, out);
}

int rk_matrix_set_raw(rk_matrix *m, int32_t raw) {
    if (!m) return RK_ERR_ARGS;
    if (m->kind != RK_FP8 && m->kind != RK_FP4)
        return fail(m->d, RK_ERR_ARGS, "rk_matrix_set_raw: only E4M3 / E2M1 products round to bfloat16");
    m->raw = raw != 0;
    return RK_OK;
}

int rk_matrix_free(rk_matrix *m) {
    if (!m) return RK_ERR_ARGS;
    rk_device *d = m->d;
    Hold hold(d->gate);
    (void)hipSetDevice(d->index);
    (void)hipStreamSynchronize(d->stream);
    (void)hipFree(m->w);
    (void)hipFree(m->scales);
    (void)hipFree(m->e8m0);
    add_used(d, -m->bytes);
    delete m;
    return RK_OK;
}

int64_t rk_matrix_bytes(const rk_matrix *m) { return m ? m->bytes : -1; }

int rk_matvecs(rk_device *d, int32_t n, rk_matrix *const *ms, float *const *outs, const float *x, int64_t cols) {
    int64_t total;
    int rc = check_products(d, n, ms, cols, &total);
    if (rc) return rc;
    if (n == 0) return RK_OK;
    if (!x || !outs) return fail(d, RK_ERR_ARGS, "rk_matvecs: null buffer");
    if (total > kMaxRows) return fail(d, RK_ERR_ARGS, "gpu: products too large for one submission");
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    hipStream_t s = d->stream;
    float *hx = d->h_stage, *hout = d->h_stage + kMaxCols;
    memcpy(hx, x, (size_t)cols * 4);
    if ((rc = scratch_acquire(d, s))) return rc;
    HIP_TRY(d, hipMemcpyAsync(d->x, hx, (size_t)cols * 4, hipMemcpyHostToDevice, s), "input copy");
    if (d->capturing) return fail(d, RK_ERR_ARGS, "rk_matvecs waits for its results: it cannot be recorded");
    std::vector<float *> douts(n);
    int64_t at = 0;
    for (int i = 0; i < n; i++) {
        douts[i] = d->out + at;
        at += ms[i]->rows;
    }
    if ((rc = enqueue_matvecs(d, n, ms, douts.data(), d->x, cols, QScratch{d->qx, d->xs, d->xsum}, s))) return rc;
    HIP_TRY(d, hipMemcpyAsync(hout, d->out, (size_t)total * 4, hipMemcpyDeviceToHost, s), "output copy");
    HIP_TRY(d, hipStreamSynchronize(s), "submit");
    at = 0;
    for (int i = 0; i < n; i++) {
        memcpy(outs[i], hout + at, (size_t)ms[i]->rows * 4);
        at += ms[i]->rows;
    }
    return RK_OK;
}

int rk_matvecs_device(rk_device *d, int32_t n, rk_matrix *const *ms, float *const *d_outs, const float *d_x,
                      int64_t cols, void *stream) {
    int64_t total;
    int rc = check_products(d, n, ms, cols, &total);
    if (rc) return rc;
    if (n == 0) return RK_OK;
    if (!d_x || !d_outs) return fail(d, RK_ERR_ARGS, "rk_matvecs_device: null buffer");
    for (int i = 0; i < n; i++)
        if (!d_outs[i]) return fail(d, RK_ERR_ARGS, "rk_matvecs_device: null output %d", i);
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    hipStream_t s = stream ? (hipStream_t)stream : d->stream;
    if (d->capturing && s != d->stream)
        return fail(d, RK_ERR_ARGS, "while recording a graph, work goes on the device's stream");
    if ((rc = scratch_acquire(d, s))) return rc;
    return enqueue_matvecs(d, n, ms, d_outs, d_x, cols, QScratch{d->qx, d->xs, d->xsum}, s);
}

int rk_matmul_t(rk_device *d, int32_t n, rk_matrix *const *ms, float *const *outs, const float *x, int64_t cols,
                int32_t tokens) {
    int64_t total;
    int rc = check_matmul(d, n, ms, cols, tokens, &total);
    if (rc) return rc;
    if (n == 0 || tokens == 0) return RK_OK;
    if (!x || !outs) return fail(d, RK_ERR_ARGS, "rk_matmul_t: null buffer");
    for (int i = 0; i < n; i++)
        if (!outs[i]) return fail(d, RK_ERR_ARGS, "rk_matmul_t: null output %d", i);
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    if (d->capturing) return fail(d, RK_ERR_ARGS, "rk_matmul_t waits for its results: it cannot be recorded");
    hipStream_t s = d->stream;
    if ((rc = scratch_acquire(d, s))) return rc;
    if ((rc = grow(d, (void **)&d->bx, d->bx_cap, cols * tokens, 4, "batch input")) ||
        (rc = grow(d, (void **)&d->bout, d->bout_cap, total * tokens, 4, "batch output")) ||
        (rc = batch_scratch(d, cols * tokens)))
        return rc;
    HIP_TRY(d, hipMemcpyAsync(d->bx, x, (size_t)(cols * tokens) * 4, hipMemcpyHostToDevice, s), "input copy");
    std::vector<float *> douts(n);
    int64_t at = 0;
    for (int i = 0; i < n; i++) {
        douts[i] = d->bout + at;
        at += ms[i]->rows * tokens;
    }
    if ((rc = enqueue_matmuls(d, n, ms, douts.data(), d->bx, cols, tokens, QScratch{d->bqx, d->bxs, d->bxsum}, s)))
        return rc;
    at = 0;
    for (int i = 0; i < n; i++) {
        HIP_TRY(d, hipMemcpyAsync(outs[i], d->bout + at, (size_t)(ms[i]->rows * tokens) * 4, hipMemcpyDeviceToHost, s),
                "output copy");
        at += ms[i]->rows * tokens;
    }
    HIP_TRY(d, hipStreamSynchronize(s), "submit");
    return RK_OK;
}

int rk_matmul_t_device(rk_device *d, int32_t n, rk_matrix *const *ms, float *const *d_outs, const float *d_x,
                       int64_t cols, int32_t tokens, void *stream) {
    int64_t total;
    int rc = check_matmul(d, n, ms, cols, tokens, &total);
    if (rc) return rc;
    if (n == 0 || tokens == 0) return RK_OK;
    if (!d_x || !d_outs) return fail(d, RK_ERR_ARGS, "rk_matmul_t_device: null buffer");
    for (int i = 0; i < n; i++)
        if (!d_outs[i]) return fail(d, RK_ERR_ARGS, "rk_matmul_t_device: null output %d", i);
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    hipStream_t s = stream ? (hipStream_t)stream : d->stream;
    if (d->capturing && s != d->stream)
        return fail(d, RK_ERR_ARGS, "while recording a graph, work goes on the device's stream");
    if ((rc = scratch_acquire(d, s))) return rc;
    if ((rc = batch_scratch(d, cols * tokens))) return rc;
    return enqueue_matmuls(d, n, ms, d_outs, d_x, cols, tokens, QScratch{d->bqx, d->bxs, d->bxsum}, s);
}

int rk_graph_begin(rk_device *d) {
    if (!d) return RK_ERR_ARGS;
    Hold hold(d->gate);
    if (d->capturing) return fail(d, RK_ERR_ARGS, "rk_graph_begin: already recording");
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    HIP_TRY(d, hipStreamSynchronize(d->stream), "graph begin");
    HIP_TRY(d, hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal), "graph begin");
    d->capturing = true;
    return RK_OK;
}

int rk_graph_end(rk_device *d, rk_graph **out) {
    if (!d || !out) return RK_ERR_ARGS;
    *out = nullptr;
    Hold hold(d->gate);
    if (!d->capturing) return fail(d, RK_ERR_ARGS, "rk_graph_end: not recording");
    d->capturing = false;
    hipGraph_t g = nullptr;
    HIP_TRY(d, hipStreamEndCapture(d->stream, &g), "graph end");
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        (void)hipGetLastError();
        return hip_fail(d, e, "graph instantiate");
    }
    rk_graph *gr = new rk_graph();
    gr->d = d;
    gr->graph = g;
    gr->exec = ex;
    *out = gr;
    return RK_OK;
}

int rk_graph_launch(rk_graph *g, int32_t times) {
    if (!g || times < 0) return RK_ERR_ARGS;
    rk_device *d = g->d;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    for (int32_t i = 0; i < times; i++) HIP_TRY(d, hipGraphLaunch(g->exec, d->stream), "graph launch");
    HIP_TRY(d, hipStreamSynchronize(d->stream), "graph wait");
    return RK_OK;
}

int rk_graph_launch_timed(rk_graph *g, int32_t times, float *ms) {
    if (!g || times < 0 || !ms) return RK_ERR_ARGS;
    rk_device *d = g->d;
    Hold hold(d->gate);
    HIP_TRY(d, hipSetDevice(d->index), "hipSetDevice");
    hipEvent_t e0 = nullptr, e1 = nullptr;
    HIP_TRY(d, hipEventCreate(&e0), "event create");
    hipError_t e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipEventRecord(e0, d->stream);
    for (int32_t i = 0; i < times && e == hipSuccess; i++) e = hipGraphLaunch(g->exec, d->stream);
    if (e == hipSuccess) e = hipEventRecord(e1, d->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, e0, e1);
    (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (e != hipSuccess) return hip_fail(d, e, "timed graph launch");
    return RK_OK;
}

int rk_graph_free(rk_graph *g) {
    if (!g) return RK_ERR_ARGS;
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
    return RK_OK;
}

int rk_profile_start(rk_device *d) {
    if (!d) return RK_ERR_ARGS;
    Hold hold(d->gate);
    d->profiling = true;
    return RK_OK;
}

int rk_profile_stop(rk_device *d, rk_profile_entry *out, int32_t cap, int32_t *n) {
    if (!d || !n || (cap > 0 && !out)) return RK_ERR_ARGS;
    Hold hold(d->gate);
    d->profiling = false;
    std::vector<rk_profile_entry> agg;
    int rc = RK_OK;
    for (auto &r : d->prof) {
        float ms = 0;
        hipError_t e = hipEventSynchronize(r.b);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.a, r.b);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            rc = hip_fail(d, e, "profile event");
        }
        size_t i = 0;
        while (i < agg.size() && strcmp(agg[i].kernel, r.kernel) != 0) i++;
        if (i == agg.size()) {
            rk_profile_entry z{};
            snprintf(z.kernel, sizeof z.kernel, "%s", r.kernel);
            agg.push_back(z);
        }
        agg[i].calls++;
        agg[i].ms += ms;
        d->event_pool.push_back(r.a);
        d->event_pool.push_back(r.b);
    }
    d->prof.clear();
    std::sort(agg.begin(), agg.end(), [](const rk_profile_entry &x, const rk_profile_entry &y) { return x.ms > y.ms; });
    *n = (int32_t)agg.size();
    for (int32_t i = 0; i < cap && i < (int32_t)agg.size(); i++) out[i] = agg[i];
    return rc;
}

}  // extern "C"
