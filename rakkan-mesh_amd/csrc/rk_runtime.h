// rk_runtime.h — internal object model of librkhip (the C-ABI is rk.h).
#pragma once
#include <hip/hip_runtime.h>

#include <condition_variable>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/rk.h"
#include "rk_kernels.h"

// The widest input and output of one product (internal/gpu/device.go:197-200).
constexpr int64_t kMaxCols = (int64_t)1 << 18;
constexpr int64_t kMaxRows = (int64_t)1 << 20;

namespace rk {
// Ownership of a device across calls: a batch holds it from begin to submit
// (internal/gpu/batch.go:126-134), possibly on different OS threads (a Go
// goroutine may move between cgo calls), so this is a flag and a condition
// variable rather than a thread-affine mutex.
class Gate {
  public:
    void acquire() {
        std::unique_lock<std::mutex> l(m_);
        cv_.wait(l, [&] { return !held_; });
        held_ = true;
    }
    void release() {
        {
            std::lock_guard<std::mutex> l(m_);
            held_ = false;
        }
        cv_.notify_one();
    }

  private:
    std::mutex m_;
    std::condition_variable cv_;
    bool held_ = false;
};

// RAII hold of a device's gate for one call.
class Hold {
  public:
    explicit Hold(Gate &g) : g_(g) { g_.acquire(); }
    ~Hold() { g_.release(); }
    Hold(const Hold &) = delete;
    Hold &operator=(const Hold &) = delete;

  private:
    Gate &g_;
};

// Where a product's quantized input lives (device pointers).
struct QScratch {
    int8_t *qx;
    float *xs;
    int32_t *xsum;
};
}  // namespace rk

// internal/gpu/device.go:204-236 Device.
struct rk_device {
    int index = 0;
    int cu = 0;
    rk_device_info info{};
    hipStream_t stream = nullptr;
    rk::Gate gate;   // held for every call on the device, and by open batches
    std::mutex mu;   // guards `used`
    int64_t used = 0;
    std::string err;
    // Scratch of the standalone products (the reference's host arena):
    // input, its Q8 form, outputs, and pinned staging for the copies.
    float *x = nullptr;
    int8_t *qx = nullptr;
    float *xs = nullptr;
    int32_t *xsum = nullptr;
    float *out = nullptr;
    float *h_stage = nullptr;
    // Scratch of the batched products (rk_matmul_t*), grown on demand:
    // quantized inputs [tokens][cols] (codes; scales and code sums per block),
    // and f32 input/output for the host-buffer call.
    int8_t *bqx = nullptr;
    float *bxs = nullptr;
    int32_t *bxsum = nullptr;
    int64_t bq_cap = 0;  // codes
    float *bx = nullptr, *bout = nullptr;
    int64_t bx_cap = 0, bout_cap = 0;  // floats
    // Device address of rk_noalloc.hip's static scratch on this device
    // (looked up at open; rk_matmul_t_device_noalloc's quantized inputs).
    void *noalloc = nullptr;
    hipEvent_t scratch_free = nullptr;
    hipStream_t scratch_stream = nullptr;  // the last stream that used the scratch
    bool scratch_stream_set = false;
    // Kernel timing (rk_profile_*): one event pair per launch while active.
    struct ProfRec {
        const char *kernel;
        hipEvent_t a, b;
    };
    bool profiling = false;
    bool capturing = false;  // the stream is recording a graph (rk_graph_*)
    std::vector<ProfRec> prof;
    std::vector<hipEvent_t> event_pool;
};

struct rk_graph {
    rk_device *d = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

// internal/gpu/device.go:543-552 Matrix.
struct rk_matrix {
    rk_device *d = nullptr;
    int32_t kind = 0;
    int64_t rows = 0, cols = 0;
    uint8_t *w = nullptr;    // codes, [rows][row bytes]
    float *scales = nullptr; // [rows][cols/32]
    // E4M3 / E2M1 matrices: E8M0 scale bytes, [ceil(rows/32)][cols/32]
    // (RK_FP8) or [rows][cols/32] (RK_FP4); raw leaves their products in
    // float32 rather than bfloat16 (device.go:548 unrounded).
    uint8_t *e8m0 = nullptr;
    int32_t raw = 0;
    int64_t bytes = 0;
};

// internal/gpu/batch.go:75-80 Vectors: a layer's norm weights and biases.
struct rk_vectors {
    rk_device *d = nullptr;
    float *buf = nullptr;
    int64_t n = 0;
    int64_t bytes = 0;
};

namespace rk {
int fail(rk_device *d, int code, const char *fmt, ...);
int hip_fail(rk_device *d, hipError_t e, const char *what);
int dev_alloc(rk_device *d, void **p, size_t bytes, const char *what);
int scratch_acquire(rk_device *d, hipStream_t s);
// internal/gpu/batch.go:221-238: Q8_0 and E4M3 inputs are not mixed in one call.
int mixed_inputs(rk_device *d, int32_t n, rk_matrix *const *ms);
int enqueue_matvecs(rk_device *d, int32_t n, rk_matrix *const *ms, float *const *outs, const float *x, int64_t cols,
                    const QScratch &q, hipStream_t s);
void add_used(rk_device *d, int64_t bytes);
// Batched products (rk_matmul_t*): the checks, and the enqueue with the
// tokens' quantized inputs in q ([tokens][cols] codes, [tokens][cols/32]
// scales and code sums).
int check_matmul(rk_device *d, int32_t n, rk_matrix *const *ms, int64_t cols, int32_t tokens, int64_t *total);
int enqueue_matmuls(rk_device *d, int32_t n, rk_matrix *const *ms, float *const *outs, const float *x, int64_t cols,
                    int32_t tokens, const QScratch &q, hipStream_t s);
// Looks up the static scratch's device address on the current device
// (rk_noalloc.hip); called by rk_device_open.
int noalloc_setup(rk_device *d);

// Times the one kernel launched in its scope when the device is profiling
// (a scope that ends without a launch records nothing).
class ProfScope {
  public:
    ProfScope(rk_device *d, hipStream_t s, const char *kernel);
    ~ProfScope();
    ProfScope(const ProfScope &) = delete;
    ProfScope &operator=(const ProfScope &) = delete;

  private:
    rk_device *d_ = nullptr;
    const char *kernel_ = nullptr;
    LaunchEvents ev_{};
};
}  // namespace rk

#define HIP_TRY(d, expr, what)                          \
    do {                                                \
        hipError_t e_ = (expr);                         \
        if (e_ != hipSuccess) {                         \
            (void)hipGetLastError();                    \
            return ::rk::hip_fail((d), e_, (what));     \
        }                                               \
    } while (0)
