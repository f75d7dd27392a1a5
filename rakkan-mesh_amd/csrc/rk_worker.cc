// rk_worker.cc — librkworker.so: the tensor broker's worker side
// (include/rk_worker.h), built with the host compiler alone. Write a request,
// read the reply, on the inherited descriptor: no device, no file opened.
#include "../../include/rk_worker.h"

#include "rk_wire.h"

using namespace rk::wire;

extern "C" int rk_tensor_call(int32_t fd, int32_t dtype, int32_t transposed, int64_t m, int64_t k, int64_t n,
                              const void *a, const void *b, void *c) {
    if (fd < 0 || !a || !b || !c || !dims_ok(m, k, n) || (transposed != 0 && transposed != 1)) return RK_ERR_ARGS;
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
