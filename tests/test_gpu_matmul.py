"""Batched products (prompt prefill on int8 MFMA) against the CPU oracle:
every (token, row) must carry the bits of that token's own product
(internal/num/quant.go:158-196, MatVecQ8/Q4 per token as
internal/llm/model.go:504-518 runs a prompt)."""
import numpy as np
import pytest

from oracle import oracle
from test_gpu_matvec import awkward, same_bits

pytestmark = pytest.mark.gpu


def same_rows(got, want, what):
    assert got.shape == want.shape, (got.shape, want.shape)
    for t in range(got.shape[0]):
        same_bits(got[t], want[t], f"{what} token {t}")


@pytest.mark.parametrize("rows,cols,tokens", [(64, 256, 64), (100, 288, 37), (16, 32, 1), (1000, 896, 130),
                                              (130, 4096, 65), (33, 768, 200)])
def test_matmul_matches_per_token_products(dev, rows, cols, tokens):
    rng = np.random.default_rng(rows * 131 + cols * 7 + tokens)
    w = awkward(rng, rows * cols, 0.05)
    x = awkward(rng, tokens * cols, 1.0).reshape(tokens, cols)
    q8, s8 = oracle.quantize8(w)
    m = dev.upload_q8(q8, s8, rows, cols)
    same_rows(dev.matmul_t([m], x)[0], oracle.matmul_q8(q8, s8, x, tokens, rows, cols), f"q8 {rows}x{cols}")
    m.free()
    q4, s4 = oracle.quantize4(w)
    m = dev.upload_q4(q4, s4, rows, cols)
    same_rows(dev.matmul_t([m], x)[0], oracle.matmul_q4(q4, s4, x, tokens, rows, cols), f"q4 {rows}x{cols}")
    m.free()
    assert dev.used == 0


def test_matmul_segments_and_formats(dev):
    """Q, K and V of a Qwen-style layer (three matrices on one input) plus a
    Q4 matrix in the same call: one launch per format."""
    rng = np.random.default_rng(5)
    cols, tokens = 896, 77
    shapes = [(896, "q8"), (128, "q8"), (128, "q8"), (300, "q4")]
    x = awkward(rng, tokens * cols, 1.0).reshape(tokens, cols)
    ms, want = [], []
    for rows, f in shapes:
        w = awkward(rng, rows * cols, 0.05)
        if f == "q8":
            q, s = oracle.quantize8(w)
            ms.append(dev.upload_q8(q, s, rows, cols))
            want.append(oracle.matmul_q8(q, s, x, tokens, rows, cols))
        else:
            q, s = oracle.quantize4(w)
            ms.append(dev.upload_q4(q, s, rows, cols))
            want.append(oracle.matmul_q4(q, s, x, tokens, rows, cols))
    got = dev.matmul_t(ms, x)
    for i, (g, wv) in enumerate(zip(got, want)):
        same_rows(g, wv, f"matrix {i}")
    # and each token equals the batch-1 path
    for t in (0, 40, 76):
        for i, g in enumerate(dev.matvecs(ms, x[t])):
            same_bits(got[i][t], g, f"matrix {i} token {t} vs matvec")
    for m in ms:
        m.free()


@pytest.mark.parametrize("tokens", [1, 2, 3, 7, 8, 9, 16, 17, 33, 64])
def test_small_batches_of_q8_rows(dev, tokens):
    """Up to 16 tokens of Q8 rows take the small-batch kernel (eight lanes a
    row, pieces of 64 blocks), and up to 64 when the 64 x 64 MFMA tiles
    would cover few CUs (every shape here): rows not a multiple of the 32 a
    workgroup owns, widths of one block, of a ragged last piece (65 and 129
    blocks) and of 4096 columns, and three matrices concatenated in one
    launch."""
    rng = np.random.default_rng(700 + tokens)
    for rows, cols in [(1, 32), (45, 2080), (130, 4096), (700, 4128), (3000, 256)]:
        w = awkward(rng, rows * cols, 0.05)
        x = awkward(rng, tokens * cols, 1.0).reshape(tokens, cols)
        q8, s8 = oracle.quantize8(w)
        m = dev.upload_q8(q8, s8, rows, cols)
        same_rows(dev.matmul_t([m], x)[0], oracle.matmul_q8(q8, s8, x, tokens, rows, cols),
                  f"{tokens} tokens {rows}x{cols}")
        m.free()
    cols = 2048
    x = awkward(rng, tokens * cols, 1.0).reshape(tokens, cols)
    ms, want = [], []
    for rows in (96, 33, 33):
        q, s = oracle.quantize8(awkward(rng, rows * cols, 0.05))
        ms.append(dev.upload_q8(q, s, rows, cols))
        want.append(oracle.matmul_q8(q, s, x, tokens, rows, cols))
    for i, (g, wv) in enumerate(zip(dev.matmul_t(ms, x), want)):
        same_rows(g, wv, f"{tokens} tokens, matrix {i}")
    for m in ms:
        m.free()
    assert dev.used == 0


@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_matmul_prefill_shapes(dev, fmt):
    """Config-4 shapes (Qwen-7B: W1 18944x3584, W2 3584x18944) over a
    prompt-sized batch; the oracle's AVX2 path (bit-identical to the scalar
    one) keeps the check to seconds."""
    rng = np.random.default_rng(11)
    tokens = 96
    for rows, cols in [(18944, 3584), (3584, 18944)]:
        n = rows * cols
        x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
        s = rng.uniform(1e-3, 1e-2, n // 32).astype(np.float32)
        if fmt == "q8":
            q = rng.integers(-127, 128, n, dtype=np.int8)
            m = dev.upload_q8(q, s, rows, cols)
            ref = lambda xt: oracle.matvec_q8_avx2(q, s, xt, rows, cols, 8)
        else:
            q = rng.integers(0, 256, n // 2, dtype=np.uint8)
            m = dev.upload_q4(q, s, rows, cols)
            ref = lambda xt: oracle.matvec_q4_avx2(q, s, xt, rows, cols, 8)
        got = dev.matmul_t([m], x)[0]
        for t in range(tokens):
            same_bits(got[t], ref(x[t]), f"{fmt} {rows}x{cols} token {t}")
        m.free()
