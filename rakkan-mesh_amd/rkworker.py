"""The worker side of the tensor broker: librkworker.so (include/rk_worker.h)
through ctypes.

This module imports ctypes, os and numpy and loads librkworker.so alone: a
host-only library that links nothing of the GPU runtime and opens no file or
device. A worker process (the reference's isolated worker, whose seccomp
allow-list has read/write on inherited descriptors but no ioctl or openat,
internal/isolate/seccomp_linux_amd64.go:10-38) imports it and loads the
library before its filter goes on, then sends its products to the node over
an inherited descriptor (internal/isolate/inherit_unix.go:10). The node side
is rkhip.Device.tensor_serve (librkhip.so).
"""
import ctypes
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "librkworker.so")
HEADER = os.path.join(os.path.dirname(PKG_DIR), "include", "rk_worker.h")

RK_OK, RK_ERR_ARGS = 0, -1
TENSOR_F32, TENSOR_I8 = 0, 1

P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
# name -> (restype, argtypes); the exported C-ABI, kept in step with rk_worker.h.
SIGNATURES = {"rk_tensor_call": (ctypes.c_int, [I32, I32, I32, I64, I64, I64, P, P, P])}

_lib = None


class RKError(RuntimeError):
    """A non-zero status of the C-ABI (rk.h's RK_ERR_* codes)."""

    def __init__(self, code, msg):
        super().__init__(f"rk error {code}: {msg}")
        self.code = code


def lib():
    """The loaded librkworker.so; raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def tensor_call(fd, a, b, transposed=False):
    """One matmul (b [k][n]) or matmul_t (b [n][k]) through the node on
    descriptor fd (rk_tensor_call), with reads and writes on fd only: f32 in
    gives f32 out, i8 in gives i32 out. Raises RKError with the node's
    status, or RK_ERR_NO_DEVICE when the node has gone away."""
    if a.dtype != b.dtype or a.dtype not in (np.float32, np.int8):
        raise RKError(RK_ERR_ARGS, "tensor call: f32 or i8 inputs of one type")
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    m, k = a.shape
    n = b.shape[0] if transposed else b.shape[1]
    if (b.shape[1] if transposed else b.shape[0]) != k:
        raise RKError(RK_ERR_ARGS, "tensor call: shapes differ")
    dt = TENSOR_F32 if a.dtype == np.float32 else TENSOR_I8
    c = np.empty((m, n), np.float32 if dt == TENSOR_F32 else np.int32)
    ptr = lambda x: x.ctypes.data_as(P)  # noqa: E731
    rc = lib().rk_tensor_call(fd, dt, int(bool(transposed)), m, k, n, ptr(a), ptr(b), ptr(c))
    if rc != RK_OK:
        raise RKError(rc, "tensor call through the broker")
    return c
