// rk_broker.hip — the node side of the rakkan_tensor_v1 matmul across the
// worker process boundary: rk_tensor_serve answers a worker's requests with
// rk_tensor_matmul's results on the device. The worker validates and charges
// gas as tenMatmul does (internal/sandbox/tensor.go:286-339) and sends the
// request with rk_tensor_call (librkworker.so, host only: the worker loads no
// GPU runtime). Wire format and descriptor I/O: rk_wire.h. Host code only:
// no kernels here.
#include <vector>

#include "rk_runtime.h"
#include "rk_wire.h"

namespace rk {
namespace {

using namespace wire;

constexpr int64_t kDefaultMaxBytes = (int64_t)1 << 30;

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
        if (q.magic != kReqMagic || q.op != kOpMatmul || es == 0 || !dims_ok(q.m, q.k, q.n) ||
            (q.transposed != 0 && q.transposed != 1) ||
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
