"""A tensor-broker worker for tests/test_gpu_broker.py, run as its own
process: it sends a fixed list of products through the node on an inherited
descriptor (rk_tensor_call, reads and writes on that descriptor only; no
device is opened here, as in the reference's seccomp worker) and saves the
results.

    python broker_worker.py <fd> <out.npz>
"""
import os
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


def main():
    import rkhip

    fd, path = int(sys.argv[1]), sys.argv[2]
    res = {name: rkhip.tensor_call(fd, a, b, t) for name, a, b, t in cases()}
    np.savez(path, **res)
    os.close(fd)


if __name__ == "__main__":
    main()
