"""The oracle's MoE feed-forward (this build's contract, after
internal/llm/dsv41/ops.go:67-74 topK and forward.go:355-413 moe). The
reference has no llama-family MoE to compare with, so its pieces are pinned
here: topK against numpy's stable sort under Go's cmp.Compare order, and
the composition against the same steps written with the oracle's pinned
primitives (MatVecQ8, softmax, silu, Recip32)."""
import numpy as np

from oracle import oracle
from oracle.model import Mat


def go_cmp_sort_desc(v):
    """Stable descending order by cmp.Compare (NaN lowest, -0 == +0)."""
    key = np.where(np.isnan(v), -np.inf, v).astype(np.float64)
    nan_rank = np.isnan(v).astype(np.int64)  # NaN after every number, even -Inf
    return np.lexsort((np.arange(v.size), -key, nan_rank))


def test_topk_is_a_stable_descending_sort():
    rng = np.random.default_rng(1)
    for trial in range(200):
        n = int(rng.integers(1, 200))
        v = rng.integers(-5, 6, n).astype(np.float32)  # many ties
        if trial % 3 == 0:
            v[rng.integers(0, n, 3)] = np.nan
        if trial % 5 == 0:
            v[rng.integers(0, n, 2)] = -0.0
        k = int(rng.integers(1, n + 1))
        want = go_cmp_sort_desc(v)[:k]
        assert list(oracle.topk(v, k)) == list(want), (v, k)


def test_moe_composition():
    """The contract's three order choices, each on inputs where the
    plausible alternative gives other bits (checked in the test, so a
    planted slip in the oracle fails it): experts added in ascending index
    (not selection order), each weight applied to the expert's hidden
    activation before W2 (not to its output), and the weights' normalising
    sum taken in selection order (not ascending)."""
    rng = np.random.default_rng(2)
    dim, hidden, experts, k = 96, 64, 12, 3
    q8 = lambda r, c: Mat(r, c, (rng.normal(0, 0.2, r * c)).astype(np.float32), "q8_0")  # noqa: E731
    router = q8(experts, dim)
    w1 = [q8(hidden, dim) for _ in range(experts)]
    w3 = [q8(hidden, dim) for _ in range(experts)]
    w2 = [q8(dim, hidden) for _ in range(experts)]
    differs = {"selection-order sum": 0, "weight on the output": 0, "ascending weight sum": 0}
    for t in range(20):
        xn = rng.normal(0, 1, dim).astype(np.float32)
        y, sel, w = oracle.moe_ffn(router, w1, w2, w3, k, xn)
        p = oracle.softmax(oracle.matvec_q8(router.q, router.scales, xn, experts, dim))
        s = oracle.topk(p, k)
        assert list(sel) == list(s)
        tot = np.float32(0)
        for e in s:
            tot = np.float32(tot + p[e])
        inv = oracle.recip32(tot)
        ww = (p[s] * inv).astype(np.float32)
        assert np.array_equal(w.view(np.uint32), ww.view(np.uint32))
        outs, outs_unweighted = {}, {}
        for e in s:
            g = oracle.matvec_q8(w1[e].q, w1[e].scales, xn, hidden, dim)
            u = oracle.matvec_q8(w3[e].q, w3[e].scales, xn, hidden, dim)
            sg = oracle.num_eval(3, g)  # silu
            gu = (sg * u).astype(np.float32)
            h = (ww[list(s).index(e)] * gu).astype(np.float32)
            outs[e] = oracle.matvec_q8(w2[e].q, w2[e].scales, h, dim, hidden)
            outs_unweighted[e] = oracle.matvec_q8(w2[e].q, w2[e].scales, gu, dim, hidden)

        def add(order, terms):
            acc = np.zeros(dim, np.float32)
            for e in order:
                acc = (acc + terms[e]).astype(np.float32)
            return acc.view(np.uint32)

        assert np.array_equal(y.view(np.uint32), add(sorted(s), outs))
        alt = {e: (ww[list(s).index(e)] * outs_unweighted[e]).astype(np.float32) for e in s}
        differs["selection-order sum"] += not np.array_equal(y.view(np.uint32), add(list(s), outs))
        differs["weight on the output"] += not np.array_equal(y.view(np.uint32), add(sorted(s), alt))
        tot_asc = np.float32(0)
        for e in sorted(s):
            tot_asc = np.float32(tot_asc + p[e])
        differs["ascending weight sum"] += not np.array_equal(ww.view(np.uint32),
                                                              (p[s] * oracle.recip32(tot_asc)).astype(np.float32).view(np.uint32))
    assert all(n > 0 for n in differs.values()), differs
