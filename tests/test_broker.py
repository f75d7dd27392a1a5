"""The worker side of the tensor broker (rk_tensor_call, librkworker.so)
against a node written here from the wire format, on the CPU: the request it
writes (header fields, operand bytes), the result it takes back, the node's
status passed through, a node that has gone away, and a worker process that
maps none of the GPU runtime, holds no GPU descriptor and runs under a filter
that refuses open and ioctl. The node side (rk_tensor_serve) on the device is
tests/test_gpu_broker.py. The reference runs the operators in a worker that
can read and write inherited descriptors but cannot open a GPU
(internal/isolate/seccomp_linux_amd64.go:10-38, inherit_unix.go:10)."""
import errno
import os
import platform
import socket
import struct
import subprocess
import sys
import threading

import numpy as np
import pytest

import broker_worker
import rkhip
import rkworker
from oracle import oracle

REQ = struct.Struct("<IIiiqqqQQ")  # magic, op, dtype, transposed, m, k, n, a_bytes, b_bytes
REP = struct.Struct("<IiQ")        # magic, status, c_bytes
REQ_MAGIC, REP_MAGIC = 0x51544B52, 0x41544B52


def recv_all(s, n):
    b = bytearray()
    while len(b) < n:
        chunk = s.recv(n - len(b))
        if not chunk:
            raise EOFError
        b += chunk
    return bytes(b)


def fake_node(sock, seen, answer):
    """Reads one request, records it, answers with answer(header) ->
    (status, c bytes)."""
    h = REQ.unpack(recv_all(sock, REQ.size))
    a = recv_all(sock, h[7])
    b = recv_all(sock, h[8])
    seen.append((h, a, b))
    status, c = answer(h)
    sock.sendall(REP.pack(REP_MAGIC, status, len(c)) + c)


def call_with(node_answer, a, b, transposed=False):
    w, n = socket.socketpair()
    seen = []
    t = threading.Thread(target=fake_node, args=(n, seen, node_answer))
    t.start()
    try:
        return rkworker.tensor_call(w.fileno(), a, b, transposed), seen
    finally:
        t.join(10)
        w.close()
        n.close()


@pytest.mark.parametrize("transposed", [False, True])
def test_request_layout_and_result(transposed):
    rng = np.random.default_rng(3)
    a = rng.normal(0, 1, (3, 5)).astype(np.float32)
    b = rng.normal(0, 1, (4, 5) if transposed else (5, 4)).astype(np.float32)
    c = np.arange(12, dtype=np.float32).reshape(3, 4) * np.float32(0.5)
    got, seen = call_with(lambda h: (0, c.tobytes()), a, b, transposed)
    (h, ab, bb), = seen
    assert h == (REQ_MAGIC, 1, rkhip.TENSOR_F32, int(transposed), 3, 5, 4, a.nbytes, b.nbytes)
    assert ab == a.tobytes() and bb == b.tobytes()
    assert np.array_equal(got.view(np.uint32), c.view(np.uint32))


def test_int8_request_and_int32_result():
    a = np.array([[1, -2, 3]], np.int8)
    b = np.array([[4], [5], [-6]], np.int8)
    c = np.array([[-24]], np.int32)
    got, seen = call_with(lambda h: (0, c.tobytes()), a, b)
    (h, ab, bb), = seen
    assert h[2] == rkhip.TENSOR_I8 and h[7] == 3 and h[8] == 3
    assert got.dtype == np.int32 and got[0, 0] == -24


@pytest.mark.parametrize("status", [rkhip.RK_ERR_ARGS, rkhip.RK_ERR_OOM, rkhip.RK_ERR_HIP])
def test_node_status_comes_back(status):
    a = np.ones((2, 2), np.float32)
    with pytest.raises(rkhip.RKError) as e:
        call_with(lambda h: (status, b""), a, a)
    assert e.value.code == status


def test_node_gone():
    """A node that closed its end: the call reports the broker as gone
    (RK_ERR_NO_DEVICE) rather than raising a signal or hanging."""
    w, n = socket.socketpair()
    n.close()
    a = np.ones((2, 2), np.float32)
    with pytest.raises(rkhip.RKError) as e:
        rkworker.tensor_call(w.fileno(), a, a)
    assert e.value.code == rkhip.RK_ERR_NO_DEVICE
    w.close()


def test_arguments_the_request_cannot_carry():
    W = rkworker.lib()
    x = np.ones(4, np.float32)
    p = x.ctypes.data
    # a type the product does not take, a dimension past 2^24, a bad transposed flag
    assert W.rk_tensor_call(0, rkhip.TENSOR_I32, 0, 2, 2, 1, p, p, p) == rkhip.RK_ERR_ARGS
    assert W.rk_tensor_call(0, rkhip.TENSOR_F32, 0, 1 << 25, 1, 1, p, p, p) == rkhip.RK_ERR_ARGS
    assert W.rk_tensor_call(0, rkhip.TENSOR_F32, 2, 1, 1, 1, p, p, p) == rkhip.RK_ERR_ARGS
    # the node side without a device
    assert rkhip.lib().rk_tensor_serve(None, 0, 0) == rkhip.RK_ERR_ARGS


GPU_RUNTIME = ("librkhip", "libamdhip64", "libhsa-runtime64", "libhsakmt", "libdrm_amdgpu", "libamd_comgr")


def test_worker_library_links_no_gpu_runtime():
    """librkworker.so needs the C library alone (its dynamic section), and
    librkhip.so no longer carries the worker's entry point."""
    dyn = subprocess.run(["readelf", "-d", rkworker.LIB_PATH], capture_output=True, text=True, check=True).stdout
    needed = [line.split("[")[1].split("]")[0] for line in dyn.splitlines() if "(NEEDED)" in line]
    assert needed and all(n.startswith(("libc.so", "libstdc++", "libgcc_s", "libm.so")) for n in needed), needed
    sym = subprocess.run(["nm", "-D", "--defined-only", rkhip.LIB_PATH], capture_output=True, text=True, check=True)
    assert " rk_tensor_call" not in sym.stdout


@pytest.mark.skipif(platform.machine() != "x86_64", reason="the worker's filter is written for x86-64")
def test_worker_process_maps_no_gpu_runtime_and_runs_under_a_filter(tmp_path):
    """A worker process (tests/broker_worker.py --seccomp --hold) sends its
    products to a node written here, which answers each with the oracle's
    product. While the worker is alive: its mappings hold librkworker.so and
    no GPU runtime library, and none of its descriptors is /dev/kfd or a
    /dev/dri node. Under its filter opening /dev/kfd fails with EPERM, and
    every product still comes back with the node's bits."""
    node, worker = socket.socketpair()
    out = tmp_path / "worker.npz"
    p = subprocess.Popen([sys.executable, broker_worker.__file__, str(worker.fileno()), str(out), "--seccomp", "--hold"],
                         pass_fds=(worker.fileno(),))
    worker.close()
    sent = {}
    try:
        for name, a, b, t in broker_worker.cases():
            h = REQ.unpack(recv_all(node, REQ.size))
            ab, bb = recv_all(node, h[7]), recv_all(node, h[8])
            a2 = np.frombuffer(ab, a.dtype).reshape(a.shape)
            b2 = np.frombuffer(bb, b.dtype).reshape(b.shape)
            c = oracle.tensor_matmul_f32(a2, b2, t) if a.dtype == np.float32 else oracle.tensor_matmul_i8(a2, b2, t)
            sent[name] = c
            node.sendall(REP.pack(REP_MAGIC, 0, c.nbytes) + c.tobytes())
        maps = open(f"/proc/{p.pid}/maps").read()
        fds = [os.readlink(f"/proc/{p.pid}/fd/{f}") for f in os.listdir(f"/proc/{p.pid}/fd")]
        node.sendall(b"x")
        assert p.wait(60) == 0
    finally:
        if p.poll() is None:
            p.kill()
        node.close()
    assert "librkworker.so" in maps
    mapped = [lib for lib in GPU_RUNTIME if lib in maps]
    assert not mapped, mapped
    assert not [f for f in fds if f.startswith(("/dev/kfd", "/dev/dri"))], fds
    got = np.load(out)
    assert int(got["kfd_open_errno"]) == errno.EPERM
    for name, c in sent.items():
        assert got[name].dtype == c.dtype and np.array_equal(got[name].view(np.uint32), c.view(np.uint32)), name
