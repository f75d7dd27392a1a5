"""The MoE feed-forward on the GPU (rk_moe_*) against the oracle's contract,
bit for bit per token: outputs, selected experts and their weights, at a
small shape, at config 5's (Qwen3-MoE: dim 2048, 128 experts of 768, top 8)
for batches of 1 and 16, and with tied router logits."""
import numpy as np
import pytest

import rkhip
from oracle import oracle
from oracle.model import Mat, Q8

pytestmark = pytest.mark.gpu


def coded(rng, rows, cols, lo=1e-3, hi=1e-2):
    q = rng.integers(-127, 128, rows * cols, dtype=np.int8)
    s = rng.uniform(lo, hi, rows * cols // 32).astype(np.float32)
    return Mat.from_codes(Q8, rows, cols, q, s)


def build(dev, rng, dim, hidden, experts, router=None):
    router = router or coded(rng, experts, dim, 1e-3, 3e-3)
    w1 = [coded(rng, hidden, dim) for _ in range(experts)]
    w3 = [coded(rng, hidden, dim) for _ in range(experts)]
    w2 = [coded(rng, dim, hidden, 1e-4, 1e-3) for _ in range(experts)]
    up = lambda m: dev.upload_q8(m.q, m.scales, m.rows, m.cols)  # noqa: E731
    g = (up(router), [up(m) for m in w1], [up(m) for m in w2], [up(m) for m in w3])
    return (router, w1, w2, w3), g


def check(dev, host, gpu, topk, xs):
    router, w1, w2, w3 = host
    moe = rkhip.Moe(dev, gpu[0], gpu[1], gpu[2], gpu[3], topk)
    y, sel, w = moe.ffn(xs)
    for t in range(xs.shape[0]):
        wy, ws, ww = oracle.moe_ffn(router, w1, w2, w3, topk, xs[t])
        assert list(sel[t]) == list(ws), f"token {t}: experts {sel[t]} vs {ws}"
        assert np.array_equal(w[t].view(np.uint32), ww.view(np.uint32)), f"token {t}: weights"
        assert np.array_equal(y[t].view(np.uint32), wy.view(np.uint32)), f"token {t}: output"
    moe.free()
    for m in [gpu[0]] + gpu[1] + gpu[2] + gpu[3]:
        m.free()


@pytest.mark.parametrize("tokens", [1, 5, 16, 40])
def test_moe_small(dev, tokens):
    rng = np.random.default_rng(tokens)
    host, gpu = build(dev, rng, 256, 128, 16)
    check(dev, host, gpu, 4, rng.normal(0, 1, (tokens, 256)).astype(np.float32))
    assert dev.used == 0


@pytest.mark.parametrize("tokens", [1, 16])
def test_moe_config5_shape(dev, tokens):
    rng = np.random.default_rng(50 + tokens)
    host, gpu = build(dev, rng, 2048, 768, 128)
    check(dev, host, gpu, 8, rng.normal(0, 1, (tokens, 2048)).astype(np.float32))
    assert dev.used == 0


@pytest.mark.parametrize("experts,topk,tokens", [(200, 8, 1), (200, 8, 16), (200, 8, 40), (64, 32, 4),
                                                  (64, 32, 5)])
def test_moe_routing_launch_shapes(dev, experts, topk, tokens):
    """More than 128 experts (a lane holds up to 16 of them), and the
    routing of up to 16 tokens with at most 128 (token, slot) pairs in one
    launch with the grouping, or one launch per token past that."""
    rng = np.random.default_rng(experts * 7 + topk + tokens)
    host, gpu = build(dev, rng, 128, 64, experts)
    check(dev, host, gpu, topk, rng.normal(0, 1, (tokens, 128)).astype(np.float32))
    assert dev.used == 0


def test_moe_tied_router_logits(dev):
    """Experts whose router rows are equal tie: the lower index is taken
    first (a stable sort), on the GPU as in the oracle."""
    rng = np.random.default_rng(7)
    experts, dim = 24, 128
    base = coded(rng, 4, dim, 1e-3, 3e-3)
    q = np.concatenate([base.q.reshape(4, dim)[i % 4] for i in range(experts)])
    s = np.concatenate([base.scales.reshape(4, dim // 32)[i % 4] for i in range(experts)])
    router = Mat.from_codes(Q8, experts, dim, q, s)
    host, gpu = build(dev, rng, dim, 64, experts, router)
    check(dev, host, gpu, 6, rng.normal(0, 1, (9, dim)).astype(np.float32))
