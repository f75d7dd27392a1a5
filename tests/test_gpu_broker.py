"""The node side of the tensor broker (rk_tensor_serve) on the MI355X: a
worker process that opens no device (as the reference's seccomp worker,
internal/isolate/seccomp_linux_amd64.go:10-38) sends its rakkan_tensor_v1
products over an inherited socket (internal/isolate/inherit_unix.go:10),
and this process answers them on the GPU. The results equal the oracle's
and the direct product's bits; malformed and oversized requests are
answered with their error and end serving."""
import errno
import os
import platform
import socket
import subprocess
import sys
import threading

import numpy as np
import pytest

import broker_worker
import rkhip
from oracle import oracle
from test_broker import REP, REQ, REQ_MAGIC, recv_all

pytestmark = pytest.mark.gpu


def bits(x):
    x = np.ascontiguousarray(x)
    return x.view(np.uint32) if x.dtype == np.float32 else x


def test_worker_products_through_the_node(dev, tmp_path):
    """The worker process loads librkworker.so alone and runs under a filter
    that refuses open and ioctl (opening /dev/kfd gives EPERM there); the
    node serves its products on the device, every result the oracle's bits."""
    node, worker = socket.socketpair()
    out = tmp_path / "res.npz"
    args = [sys.executable, broker_worker.__file__, str(worker.fileno()), str(out)]
    if platform.machine() == "x86_64":
        args.append("--seccomp")
    p = subprocess.Popen(args, pass_fds=(worker.fileno(),))
    worker.close()
    err = []

    def serve():
        try:
            dev.tensor_serve(node.fileno())  # until the worker closes its end
        except Exception as e:  # noqa: BLE001 (reported below)
            err.append(e)

    t = threading.Thread(target=serve)
    t.start()
    try:
        rc = p.wait(timeout=120)
    except subprocess.TimeoutExpired:
        p.kill()
        rc = p.wait()
    t.join(60)
    node.close()
    assert not t.is_alive() and not err, err
    assert rc == 0
    res = np.load(out)
    if platform.machine() == "x86_64":
        assert int(res["kfd_open_errno"]) == errno.EPERM
    for name, a, b, tr in broker_worker.cases():
        want = oracle.tensor_matmul_f32(a, b, tr) if a.dtype == np.float32 else oracle.tensor_matmul_i8(a, b, tr)
        assert np.array_equal(bits(res[name]), bits(want)), name
        assert np.array_equal(bits(dev.tensor_matmul(a, b, transposed=tr)), bits(res[name])), name
    assert dev.used == 0


def serve_one_bad(dev, request, max_bytes=0):
    """Sends `request` (header and payload bytes) from a thread; returns the
    node's reply status and the error serving ended with."""
    node, worker = socket.socketpair()
    got = []

    def send():
        worker.sendall(request)
        got.append(REP.unpack(recv_all(worker, REP.size)))

    t = threading.Thread(target=send)
    t.start()
    with pytest.raises(rkhip.RKError) as e:
        dev.tensor_serve(node.fileno(), max_bytes)
    t.join(30)
    node.close()
    worker.close()
    return got[0][1], e.value.code


def test_malformed_request_is_answered_and_ends_serving(dev):
    a = np.ones(4, np.float32).tobytes()
    status, code = serve_one_bad(dev, REQ.pack(0xDEADBEEF, 1, rkhip.TENSOR_F32, 0, 2, 2, 1, 16, 8) + a + a[:8])
    assert status == code == rkhip.RK_ERR_ARGS
    # sizes that do not match the dimensions
    status, code = serve_one_bad(dev, REQ.pack(REQ_MAGIC, 1, rkhip.TENSOR_F32, 0, 2, 2, 1, 12, 8) + a)
    assert status == code == rkhip.RK_ERR_ARGS
    # an i32 product (tenMatmul refuses i32 inputs)
    status, code = serve_one_bad(dev, REQ.pack(REQ_MAGIC, 1, rkhip.TENSOR_I32, 0, 1, 1, 1, 4, 4) + a[:8])
    assert status == code == rkhip.RK_ERR_ARGS


def test_request_over_the_byte_limit(dev):
    m = k = n = 4
    payload = np.ones(m * k + k * n, np.float32).tobytes()
    status, code = serve_one_bad(dev, REQ.pack(REQ_MAGIC, 1, rkhip.TENSOR_F32, 0, m, k, n, 64, 64) + payload,
                                 max_bytes=128)
    assert status == code == rkhip.RK_ERR_OOM
