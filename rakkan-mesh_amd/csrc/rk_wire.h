// rk_wire.h — the tensor broker's wire format and descriptor I/O, shared by
// the node side (rk_tensor_serve in librkhip.so) and the worker side
// (rk_tensor_call in librkworker.so). Host code only: no HIP header, so the
// worker's library links nothing of the GPU runtime.
//
// The reference runs the tensor operators in an isolated worker whose
// seccomp allow-list has read/write on inherited descriptors but no ioctl or
// openat (internal/isolate/seccomp_linux_amd64.go:10-38); the node process
// owns the device and serves the worker's products over a descriptor the
// worker inherits (internal/isolate/inherit_unix.go:10).
//
// Little-endian. A request is a 56-byte header then a's and b's bytes; a
// reply is a 16-byte header then, for status 0, c's bytes:
//
//   request: u32 magic 'RKTQ', u32 op (1: matmul), i32 dtype, i32 transposed,
//            i64 m, i64 k, i64 n, u64 a_bytes, u64 b_bytes
//   reply:   u32 magic 'RKTA', i32 status, u64 c_bytes
#pragma once
#include <errno.h>
#include <stddef.h>
#include <stdint.h>
#include <sys/socket.h>
#include <unistd.h>

#include "../../include/rk.h"

namespace rk {
namespace wire {

constexpr uint32_t kReqMagic = 0x51544B52u;  // "RKTQ"
constexpr uint32_t kRepMagic = 0x41544B52u;  // "RKTA"
constexpr uint32_t kOpMatmul = 1;
constexpr int64_t kMaxDim = (int64_t)1 << 24;  // internal/sandbox/tensor.go:60 maxTensorDim

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

// Whole-buffer read, retrying short transfers and EINTR: 1 done, 0 end of
// stream before the first byte, -1 error or a stream that ends part way.
inline int read_all(int fd, void *p, size_t n) {
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

// Whole-buffer write. A socket is written with MSG_NOSIGNAL, so a peer that
// has gone away is an error here rather than a SIGPIPE; other descriptors
// with write.
inline bool write_all(int fd, const void *p, size_t n) {
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
inline int64_t elem_bytes(int32_t dtype) { return dtype == RK_TENSOR_F32 ? 4 : dtype == RK_TENSOR_I8 ? 1 : 0; }

inline bool dims_ok(int64_t m, int64_t k, int64_t n) {
    return m >= 1 && m <= kMaxDim && k >= 1 && k <= kMaxDim && n >= 1 && n <= kMaxDim;
}

}  // namespace wire
}  // namespace rk
