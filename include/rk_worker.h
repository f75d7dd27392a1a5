/*
 * rk_worker.h — the worker side of the tensor broker: librkworker.so.
 *
 * A host-only library (plain C++, no HIP): it links nothing of the GPU
 * runtime and opens no file or device, so the reference's isolated worker,
 * whose seccomp allow-list has read/write on inherited descriptors but no
 * ioctl or openat (internal/isolate/seccomp_linux_amd64.go:10-38), can load
 * it before its filter goes on and call it after. The node side is
 * rk_tensor_serve in librkhip.so (rk.h); the wire format is
 * rakkan-mesh_amd/csrc/rk_wire.h. Status codes and tensor types are rk.h's.
 */
#ifndef RK_WORKER_H
#define RK_WORKER_H

#include "rk.h"

#ifdef __cplusplus
extern "C" {
#endif

/* internal/sandbox/tensor.go:286-339 (tenMatmul's body, across the worker
 * boundary): one product through the node on fd, with write and read on fd
 * only. Returns the node's status for the request, RK_ERR_ARGS for
 * arguments the request cannot carry (a type other than RK_TENSOR_F32 /
 * RK_TENSOR_I8, a dimension outside 1..2^24, transposed not 0 or 1, a null
 * buffer), or RK_ERR_NO_DEVICE when the stream is closed or broken. */
int rk_tensor_call(int32_t fd, int32_t dtype, int32_t transposed, int64_t m, int64_t k, int64_t n, const void *a,
                   const void *b, void *c);

#ifdef __cplusplus
}
#endif

#endif
