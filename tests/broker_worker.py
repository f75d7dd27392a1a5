"""A tensor-broker worker for tests/test_gpu_broker.py and tests/test_broker.py,
run as its own process: it sends a fixed list of products through the node on
an inherited descriptor and saves the results.

    python broker_worker.py <fd> <out.npz> [--seccomp] [--hold]

It imports rkworker alone (librkworker.so: host code, no GPU runtime) and
writes and reads the descriptor only, as the reference's isolated worker does
(internal/isolate/seccomp_linux_amd64.go:10-38, inherit_unix.go:10).
--seccomp: before the first product, a seccomp filter makes open, openat,
openat2, creat and ioctl fail with EPERM (the reference's allow-list has
neither), and the worker records what opening /dev/kfd then gives.
--hold: after the last product the worker waits for one byte from the node,
so the node can look at the live process (its mappings and descriptors).
"""
import errno
import os
import platform
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "rakkan-mesh_amd"))


def cases():
    """(name, a, b, transposed): f32 and i8 matmul / matmul_t, with the
    operands of tensor_test.go's kinds (signs, zeros, a long k)."""
    rng = np.random.default_rng(12)
    out = []
    for i, (m, k, n) in enumerate([(3, 5, 4), (17, 300, 9), (64, 64, 64)]):
        a = rng.normal(0, 1, (m, k)).astype(np.float32)
        b = rng.normal(0, 1, (k, n)).astype(np.float32)
        out.append((f"f32_{i}", a, b, False))
        out.append((f"f32t_{i}", a, np.ascontiguousarray(b.T), True))
        ai = rng.integers(-128, 128, (m, k), dtype=np.int8)
        bi = rng.integers(-128, 128, (k, n), dtype=np.int8)
        out.append((f"i8_{i}", ai, bi, False))
        out.append((f"i8t_{i}", ai, np.ascontiguousarray(bi.T), True))
    return out


def install_filter():
    """A seccomp-BPF filter (x86-64): open (2), openat (257), openat2 (437),
    creat (85) and ioctl (16) return EPERM, anything else goes through; on
    another architecture every call returns EPERM."""
    import ctypes

    class Insn(ctypes.Structure):
        _fields_ = [("code", ctypes.c_ushort), ("jt", ctypes.c_ubyte), ("jf", ctypes.c_ubyte),
                    ("k", ctypes.c_uint32)]

    class Prog(ctypes.Structure):
        _fields_ = [("len", ctypes.c_ushort), ("filter", ctypes.POINTER(Insn))]

    ld_abs, jeq, ret = 0x20, 0x15, 0x06  # BPF_LD|W|ABS, BPF_JMP|JEQ|K, BPF_RET|K
    allow, deny = 0x7FFF0000, 0x00050000 | errno.EPERM  # SECCOMP_RET_ALLOW, SECCOMP_RET_ERRNO
    nrs = [2, 257, 437, 85, 16]
    ins = [Insn(ld_abs, 0, 0, 4), Insn(jeq, 1, 0, 0xC000003E), Insn(ret, 0, 0, deny), Insn(ld_abs, 0, 0, 0)]
    for i, nr in enumerate(nrs):
        ins.append(Insn(jeq, len(nrs) - i, 0, nr))  # to the last instruction
    ins += [Insn(ret, 0, 0, allow), Insn(ret, 0, 0, deny)]
    arr = (Insn * len(ins))(*ins)
    prog = Prog(len(ins), arr)
    libc = ctypes.CDLL(None, use_errno=True)
    if libc.prctl(38, 1, 0, 0, 0) != 0:  # PR_SET_NO_NEW_PRIVS
        raise OSError(ctypes.get_errno(), "PR_SET_NO_NEW_PRIVS")
    if libc.prctl(22, 2, ctypes.byref(prog), 0, 0) != 0:  # PR_SET_SECCOMP, SECCOMP_MODE_FILTER
        raise OSError(ctypes.get_errno(), "PR_SET_SECCOMP")


def main():
    import rkworker

    fd, path = int(sys.argv[1]), sys.argv[2]
    flags = set(sys.argv[3:])
    rkworker.lib()  # loaded before any filter, as the worker starts
    todo = cases()
    out = open(path, "wb")  # the results' file, opened before any filter
    res = {}
    if "--seccomp" in flags:
        if platform.machine() != "x86_64":
            raise SystemExit("the filter is written for x86-64")
        install_filter()
        try:
            os.close(os.open("/dev/kfd", os.O_RDWR))
            res["kfd_open_errno"] = np.array(0)
        except OSError as e:
            res["kfd_open_errno"] = np.array(e.errno)
    for name, a, b, t in todo:
        res[name] = rkworker.tensor_call(fd, a, b, t)
    if "--hold" in flags:
        os.read(fd, 1)
    np.savez(out, **res)
    out.close()
    os.close(fd)


if __name__ == "__main__":
    main()
