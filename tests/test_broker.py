"""The worker side of the tensor broker (rk_tensor_call) against a node
written here from the wire format, on the CPU: the request it writes (header
fields, operand bytes), the result it takes back, the node's status passed
through, and a node that has gone away. The node side (rk_tensor_serve) on
the device is tests/test_gpu_broker.py. The reference runs the operators in
a worker that can read and write inherited descriptors but cannot open a
GPU (internal/isolate/seccomp_linux_amd64.go:10-38)."""
import socket
import struct
import threading

import numpy as np
import pytest

import rkhip

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
        return rkhip.tensor_call(w.fileno(), a, b, transposed), seen
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
        rkhip.tensor_call(w.fileno(), a, a)
    assert e.value.code == rkhip.RK_ERR_NO_DEVICE
    w.close()


def test_arguments_the_request_cannot_carry():
    L = rkhip.lib()
    x = np.ones(4, np.float32)
    p = x.ctypes.data
    # a type the product does not take, a dimension past 2^24, a bad transposed flag
    assert L.rk_tensor_call(0, rkhip.TENSOR_I32, 0, 2, 2, 1, p, p, p) == rkhip.RK_ERR_ARGS
    assert L.rk_tensor_call(0, rkhip.TENSOR_F32, 0, 1 << 25, 1, 1, p, p, p) == rkhip.RK_ERR_ARGS
    assert L.rk_tensor_call(0, rkhip.TENSOR_F32, 2, 1, 1, 1, p, p, p) == rkhip.RK_ERR_ARGS
    # the node side without a device
    assert L.rk_tensor_serve(None, 0, 0) == rkhip.RK_ERR_ARGS
