// rk_broker.hip — the rakkan_tensor_v1 matmul across the worker process
// boundary. The reference runs the tensor operators in an isolated worker
// whose seccomp allow-list has read/write on inherited descriptors but no
// ioctl or openat (internal/isolate/seccomp_linux_amd64.go:10-38), so the
// worker cannot open a GPU. The node process owns the device and serves the
// worker's products over a descriptor the worker inherits
// (internal/isolate/inherit_unix.go:10): the worker validates and charges
// gas as tenMatmul does (internal/sandbox/tensor.go:286-339), then sends
// the request; the node answers with rk_tensor_matmul's result.
//
// Wire format, little-endian. A request is a 56-byte header then a's and
// b's bytes; a reply is a 16-byte header then, for status 0, c's bytes:
//
//   request: u32 magic 'RKTQ', u32 op (1: matmul), i32 dtype, i32 transposed,
//            i64 m, i64 k, i64 n, u64 a_bytes, u64 b_bytes
//   reply:   u32 magic 'RKTA', i32 status, u64 c_bytes
//
// Host code only: no kernels here.
#include <errno.h>
#include <string.h>
#include <sys/socket.h>
#include <unistd.h>

#include <vector>

#include "rk_runtime.h"

namespace rk {
namespace {

constexpr uint32_t kReqMagic = 0x51544B52u;  // "RKTQ"
constexpr uint32_t kRepMagic = 0x41544B52u;  // "RKTA"
constexpr uint32_t kOpMatmul = 1;
constexpr int64_t kMaxDim = (int64_t)1 << 24;       // tensor.go:60 maxTensorDim
constexpr int64_t kDefaultMaxBytes = (int64_t)1 << 30;

struct Req {
    uint32_t magic, op;
    int32_t dtype, transposed;
    int64_t m, k, n;
    uint64_t a_bytes, b_bytes;
};
static_assert(sizeof(Req) == 56, "request header layout");

struct Rep {
    uint32_t magic;
    int32_t status;
    uint64_t c_bytes;
};
static_assert(sizeof(Rep) == 16, "reply header layout");

// Whole-buffer I/O on a descriptor, retrying short transfers and EINTR.
// read_all: 1 done, 0 end of stream before the first byte, -1 error or a
// stream that ends part way.
int read_all(int fd, void *p, size_t n) {
    char *c = static_cast<char *>(p);
    size_t got = 0;
    while (got < n) {
        const ssize_t r = read(fd, c + got, n - got);
        if (r < 0 && errno == EINTR) continue;
        if (r < 0) return -1;
        if (r == 0) return got == 0 ? 0 : -1;
        got += (size_t)r;
    }
    return 1;
}

// (a socket is written with MSG_NOSIGNAL, so a peer that has gone away is
// an error here rather than a SIGPIPE; other descriptors with write)
bool write_all(int fd, const void *p, size_t n) {
    const char *c = static_cast<const char *>(p);
    size_t put = 0;
    bool sock = true;
    while (put < n) {
        ssize_t w = sock ? send(fd, c + put, n - put, MSG_NOSIGNAL) : write(fd, c + put, n - put);
        if (w < 0 && sock && errno == ENOTSOCK) {
            sock = false;
            continue;
        }
        if (w < 0 && errno == EINTR) continue;
        if (w <= 0) return false;
        put += (size_t)w;
    }
    return true;
}

// Bytes of an input element; 0 for the types the product does not take.
int64_t elem_bytes(int32_t dtype) { return dtype == RK_TENSOR_F32 ? 4 : dtype == RK_TENSOR_I8 ? 1 : 0; }

bool reply(int fd, int32_t status, const void *c, uint64_t c_bytes) {
    const Rep r{kRepMagic, status, status == RK_OK ? c_bytes : 0};
    return write_all(fd, &r, sizeof r) && (status != RK_OK || c_bytes == 0 || write_all(fd, c, c_bytes));
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" int rk_tensor_serve(rk_device *d, int32_t fd, int64_t max_bytes) {
    if (!d || fd < 0 || max_bytes < 0) return RK_ERR_ARGS;
    const int64_t cap = max_bytes ? max_bytes : kDefaultMaxBytes;
    std::vector<char> a, b, c;
    for (;;) {
        Req q;
        const int got = read_all(fd, &q, sizeof q);
        if (got == 0) return RK_OK;  // the worker closed its end
        if (got < 0) return fail(d, RK_ERR_HIP, "rk_tensor_serve: broken request stream");
        // A request whose header does not describe its own payload cannot be
        // skipped safely: answer it and drop the stream.
        const int64_t es = elem_bytes(q.dtype);
        const bool dims_ok = q.m >= 1 && q.m <= kMaxDim && q.k >= 1 && q.k <= kMaxDim && q.n >= 1 && q.n <= kMaxDim;
        if (q.magic != kReqMagic || q.op != kOpMatmul || es == 0 || !dims_ok || (q.transposed != 0 && q.transposed != 1) ||
            q.a_bytes != (uint64_t)(q.m * q.k * es) || q.b_bytes != (uint64_t)(q.k * q.n * es)) {
            (void)reply(fd, RK_ERR_ARGS, nullptr, 0);
            return fail(d, RK_ERR_ARGS, "rk_tensor_serve: malformed request (magic, op, dtype, dimensions or sizes)");
        }
        const uint64_t c_bytes = (uint64_t)(q.m * q.n * 4);
        if ((double)q.a_bytes + (double)q.b_bytes + (double)c_bytes > (double)cap) {
            (void)reply(fd, RK_ERR_OOM, nullptr, 0);
            return fail(d, RK_ERR_OOM, "rk_tensor_serve: request over the broker's byte limit");
        }
        a.resize(q.a_bytes);
        b.resize(q.b_bytes);
        c.resize(c_bytes);
        if (read_all(fd, a.data(), a.size()) != 1 || read_all(fd, b.data(), b.size()) != 1)
            return fail(d, RK_ERR_HIP, "rk_tensor_serve: request stream ended inside a payload");
        const int rc = rk_tensor_matmul(d, q.dtype, q.transposed, q.m, q.k, q.n, a.data(), b.data(), c.data());
        if (!reply(fd, rc, c.data(), c_bytes)) return fail(d, RK_ERR_HIP, "rk_tensor_serve: reply stream broken");
    }
}

extern "C" int rk_tensor_call(int32_t fd, int32_t dtype, int32_t transposed, int64_t m, int64_t k, int64_t n,
                              const void *a, const void *b, void *c) {
    if (fd < 0 || !a || !b || !c || m < 1 || k < 1 || n < 1 || m > kMaxDim || k > kMaxDim || n > kMaxDim ||
        (transposed != 0 && transposed != 1))
        return RK_ERR_ARGS;
    const int64_t es = elem_bytes(dtype);
    if (es == 0) return RK_ERR_ARGS;
    const Req q{kReqMagic, kOpMatmul, dtype, transposed, m, k, n, (uint64_t)(m * k * es), (uint64_t)(k * n * es)};
    if (!write_all(fd, &q, sizeof q) || !write_all(fd, a, q.a_bytes) || !write_all(fd, b, q.b_bytes))
        return RK_ERR_NO_DEVICE;
    Rep r;
    if (read_all(fd, &r, sizeof r) != 1 || r.magic != kRepMagic) return RK_ERR_NO_DEVICE;
    if (r.status != RK_OK) return r.status;
    if (r.c_bytes != (uint64_t)(m * n * 4) || read_all(fd, c, r.c_bytes) != 1) return RK_ERR_NO_DEVICE;
    return RK_OK;
}
