"""Config 5's decoder stack: layers whose feed-forward is a mixture of
experts (the build's contract, after internal/llm/dsv41/forward.go:355-413
and ops.go:67-74), with Qwen3 attention (QK-norm, q_dim != dim), decoded
at batch 1 (the single-sequence stage, one recorded graph per token) and as
several independent sequences at once (rk_stage_seqs_*, each sequence with
its own prompt length, position and caches; the selected experts' rows read
once per step for all the tokens that chose them). Every logit of every
step is compared bit for bit with the oracle's generation of that sequence
alone (oracle/rk_oracle.c rko_forward with rko_moe_ffn)."""
import os

import numpy as np
import pytest

import rkhip
from oracle import oracle
from oracle.model import Config, Layer, Mat, Model, Moe, Q8
from test_gpu_fused_stage import oracle_generate, same_bits

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))


def codes(rng, rows, cols, lo, hi):
    """A Q8 matrix of random codes (never -128) and scales U(lo, hi)."""
    q = rng.bit_generator.random_raw((rows * cols + 7) // 8).view(np.int8)[:rows * cols].copy()
    q[q == -128] = -127
    return Mat.from_codes(Q8, rows, cols, q, rng.uniform(lo, hi, rows * cols // 32).astype(np.float32))


def moe_model(c, experts, ehidden, topk, seed, lo=1e-4, hi=1e-3, router_scale=(1e-3, 1e-2)):
    """Random codes: Q8 attention matrices, a Q8 router per layer (scaled so
    the routing spreads over the experts) and Q8 experts; norm weights
    N(1, 0.1); Q8 embedding shared with the classifier."""
    rng = np.random.default_rng(seed)
    m = Model.__new__(Model)
    m.c = c
    d, q, kv, hs = c.dim, c.q_dim(), c.kv_dim(), c.head_size()
    m.embed = codes(rng, c.vocab, d, lo, hi)
    m.wcls = m.embed
    m.rms_final = rng.normal(1, 0.1, d).astype(np.float32)
    m.layers = []
    for _ in range(c.layers):
        ly = Layer()
        ly.rms_att = rng.normal(1, 0.1, d).astype(np.float32)
        ly.rms_ffn = rng.normal(1, 0.1, d).astype(np.float32)
        if c.qk_norm:
            ly.q_norm, ly.k_norm = (rng.normal(1, 0.1, hs).astype(np.float32) for _ in range(2))
        if c.qkv_bias:
            ly.bq, ly.bk, ly.bv = (rng.normal(0, 0.5, n).astype(np.float32) for n in (q, kv, kv))
        for n, (rows, cols) in {"wq": (q, d), "wk": (kv, d), "wv": (kv, d), "wo": (d, q)}.items():
            setattr(ly, n, codes(rng, rows, cols, lo, hi))
        router = codes(rng, experts, d, *router_scale)
        w1 = [codes(rng, ehidden, d, lo, hi) for _ in range(experts)]
        w3 = [codes(rng, ehidden, d, lo, hi) for _ in range(experts)]
        w2 = [codes(rng, d, ehidden, lo, hi) for _ in range(experts)]
        ly.moe = Moe(router, w1, w2, w3, topk)
        m.layers.append(ly)
    return m


class GpuModel:
    """The model's matrices on the device, its MoE handles, and stages."""

    def __init__(self, dev, m):
        self.dev, self.m, self.mats, self.moes = dev, m, [], []
        up = lambda mt: self._keep(dev.upload(mt.kind, mt.rows, mt.cols, mt.q, mt.scales))  # noqa: E731
        self.layers = []
        for ly in m.layers:
            d = {n: up(getattr(ly, n)) for n in ("wq", "wk", "wv", "wo")}
            for n in Layer.VECS:
                d[n] = getattr(ly, n)
            mo = ly.moe
            moe = rkhip.Moe(dev, up(mo.router), [up(w) for w in mo.w1], [up(w) for w in mo.w2],
                            [up(w) for w in mo.w3], mo.topk)
            self.moes.append(moe)
            d["moe"] = moe
            self.layers.append(d)
        self.emb = up(m.embed)

    def _keep(self, mt):
        self.mats.append(mt)
        return mt

    def stage(self, ctx, seqs=1):
        c = self.m.c
        cos, sin = self.m.rope(ctx)
        st = rkhip.Stage(self.dev, c.dim, c.hidden, c.heads, c.kv_heads, ctx, self.layers, cos, sin,
                         head_dim=c.head_dim, norm_eps=float(c.eps()), qkv_bias=c.qkv_bias, qk_norm=c.qk_norm,
                         seqs=seqs)
        st.set_head(self.emb, self.emb, self.m.rms_final)
        return st

    def free(self):
        for mo in self.moes:
            mo.free()
        for mt in self.mats:
            mt.free()


def check_batch1(g, prompt, steps, ctx):
    want_t, want_l = oracle_generate(g.m, prompt, steps, ctx)
    st = g.stage(ctx)
    st.generate_start(prompt)
    if len(prompt) > 1:
        st.generate_run(len(prompt) - 1)  # the prompt: the batched path (MoE over many tokens)
    for k in range(steps):
        same_bits(st.generate_run(1, want_logits=True)[0], want_l[k], f"batch 1, step {k}")
    assert list(st.tokens(len(prompt), steps)) == want_t
    st.free()


def check_seqs(g, prompts, steps, ctx):
    want = [oracle_generate(g.m, p, steps, ctx) for p in prompts]
    st = g.stage(ctx, seqs=len(prompts))
    st.seqs_start(prompts)
    lg = st.seqs_run(steps, want_logits=True)
    for z, (wt, wl) in enumerate(want):
        for k in range(steps):
            same_bits(lg[k, z], wl[k], f"sequence {z} (prompt {len(prompts[z])}), step {k}")
        assert list(st.seqs_tokens(z, len(prompts[z]), steps)) == wt, f"sequence {z} tokens"
    st.free()


SMALL = Config(dim=64, hidden=64, layers=2, heads=4, kv_heads=2, vocab=50, seq_len=96, head_dim=32, qk_norm=True,
               rope_theta=1e6, norm_eps=1e-6, dtype="q8_0")


def test_moe_stage_small_batch1_and_sequences(dev):
    m = moe_model(SMALL, experts=12, ehidden=64, topk=3, seed=1, lo=1e-3, hi=1e-2, router_scale=(1e-2, 5e-2))
    g = GpuModel(dev, m)
    try:
        with oracle.matvec_threads(THREADS):
            check_batch1(g, [1, 5, 9, 2, 7, 30, 11], 12, 96)
            rng = np.random.default_rng(5)
            prompts = [[int(t) for t in rng.integers(0, 50, n)] for n in (1, 2, 9, 30, 17)]
            check_seqs(g, prompts, 10, 96)
    finally:
        g.free()
    assert dev.used == 0


def test_moe_stage_expert_hidden_over_2048(dev):
    """An expert hidden width of 2080 (over 64 blocks a lane group of eight
    holds): one token's W2 rows then go through the general down kernel,
    reading the grouping that the W1/W3 launch's lead workgroup wrote, in
    place of the one-token down kernel. One sequence, then two (the grouped
    path of several tokens), every logit against the oracle."""
    m = moe_model(SMALL, experts=6, ehidden=2080, topk=2, seed=6, lo=1e-3, hi=1e-2, router_scale=(1e-2, 5e-2))
    g = GpuModel(dev, m)
    try:
        with oracle.matvec_threads(THREADS):
            check_batch1(g, [4, 9, 1], 6, 32)
            check_seqs(g, [[2, 8], [5]], 4, 32)
    finally:
        g.free()
    assert dev.used == 0


def test_profiling_a_qk_norm_prompt(dev):
    """Per-launch timing over a prompt of a QK-norm stage: the batched path
    opens a timing scope for the fused norm-and-scores launch, which it then
    declines (no launch), and times the separate norm and scores launches
    instead. The declined scope records nothing, so the readout holds only
    launches that ran, one of each per layer."""
    m = moe_model(SMALL, experts=12, ehidden=64, topk=3, seed=1, lo=1e-3, hi=1e-2, router_scale=(1e-2, 5e-2))
    g = GpuModel(dev, m)
    try:
        st = g.stage(96)
        st.generate_start([1, 5, 9, 2, 7, 30, 11])
        dev.profile_start()
        st.generate_run(6)  # the prompt's first six positions: one batch
        prof = dev.profile_stop()
        st.free()
    finally:
        g.free()
    layers = SMALL.layers
    assert prof["qknorm_rope"][0] == layers and prof["att_scores"][0] == layers, prof
    assert all(calls > 0 and ms >= 0.0 for calls, ms in prof.values()), prof
    assert dev.used == 0


@pytest.mark.parametrize("dim,experts,ehidden,topk,lo,hi", [(2048, 16, 64, 16, 2e-4, 2e-3),
                                                        (512, 32, 2048, 2, 5e-4, 5e-3),
                                                        (64, 512, 32, 4, 1e-3, 1e-2)])
def test_moe_stage_one_launch_limits(dev, dim, experts, ehidden, topk, lo, hi):
    """A decode step's whole feed-forward in one launch at the edges of the
    shapes it takes: inputs 2048 wide with 16 experts a token (four output
    rows of each a down workgroup), an expert hidden width of 2048 (eight
    W2 blocks a lane), and 512 experts (the routing's general ranks). One
    generation each over two layers, every logit against the oracle."""
    c = Config(dim=dim, hidden=64, layers=2, heads=4, kv_heads=2, vocab=50, seq_len=64, head_dim=32, qk_norm=True,
               rope_theta=1e6, norm_eps=1e-6, dtype="q8_0")
    m = moe_model(c, experts=experts, ehidden=ehidden, topk=topk, seed=9, lo=lo, hi=hi, router_scale=(1e-2, 5e-2))
    g = GpuModel(dev, m)
    try:
        with oracle.matvec_threads(THREADS):
            check_batch1(g, [3, 1, 4], 6, 64)
    finally:
        g.free()
    assert dev.used == 0


def test_moe_stage_many_experts(dev):
    """200 experts, top 8 (a lane of the routing holds up to 16 experts):
    one sequence, then three."""
    m = moe_model(SMALL, experts=200, ehidden=32, topk=8, seed=4, lo=1e-3, hi=1e-2, router_scale=(1e-2, 5e-2))
    g = GpuModel(dev, m)
    try:
        with oracle.matvec_threads(THREADS):
            check_batch1(g, [3, 1, 4, 1, 5], 8, 64)
            check_seqs(g, [[2, 7], [1, 8, 2, 8], [18]], 6, 64)
    finally:
        g.free()
    assert dev.used == 0


def test_moe_stage_sequences_reuse_and_one_sequence_stage(dev):
    """A stage of several sequences started twice (the second start
    overwrites every sequence's prompt and position), and a stage of one
    sequence driven through rk_stage_seqs_*: the same logits as alone."""
    m = moe_model(SMALL, experts=8, ehidden=32, topk=2, seed=2, lo=1e-3, hi=1e-2, router_scale=(1e-2, 5e-2))
    g = GpuModel(dev, m)
    try:
        with oracle.matvec_threads(THREADS):
            st = g.stage(64, seqs=3)
            st.seqs_start([[3, 4], [5], [6, 7, 8]])
            st.seqs_run(5)
            st.free()
            check_seqs(g, [[9, 1, 2, 3], [4, 4], [40]], 6, 64)
            check_seqs(g, [[2, 7, 1, 8, 2, 8]], 6, 64)
    finally:
        g.free()
    assert dev.used == 0


CONFIG5 = Config(dim=2048, hidden=768, layers=2, heads=32, kv_heads=4, vocab=151936, seq_len=64, head_dim=128,
                 qk_norm=True, rope_theta=1e6, norm_eps=1e-6, dtype="q8_0")


def test_config5_shape_batch1_and_16_sequences(dev):
    """Config 5's layer shape (dim 2048, 32 q / 4 kv heads of 128, QK-norm,
    128 experts of 768, top 8) over two layers with a 151936-token head: a
    batch-1 generation, then 16 independent sequences with prompts of 1 to
    31 tokens, every logit of every step bit for bit."""
    m = moe_model(CONFIG5, experts=128, ehidden=768, topk=8, seed=3, lo=2e-5, hi=2e-4, router_scale=(2e-4, 2e-3))
    g = GpuModel(dev, m)
    try:
        with oracle.matvec_threads(THREADS):
            check_batch1(g, [11, 7000, 123, 99, 5, 151935], 6, 64)
            rng = np.random.default_rng(7)
            prompts = [[int(t) for t in rng.integers(0, CONFIG5.vocab, 1 + 2 * z)] for z in range(16)]
            check_seqs(g, prompts, 4, 64)
    finally:
        g.free()
    assert dev.used == 0


def test_moe_stats_count_each_groupings_experts(dev):
    """rk_stage_moe_stats: one grouping a MoE layer a batched step. Two
    sequences with the same prompt choose the same experts at every layer
    and step, so each grouping holds exactly top-k experts; different
    prompts hold between top-k and min(experts, 2·top-k)."""
    m = moe_model(SMALL, experts=12, ehidden=64, topk=3, seed=1, lo=1e-3, hi=1e-2, router_scale=(1e-2, 5e-2))
    g = GpuModel(dev, m)
    steps = 6
    try:
        for prompts, same in (([[3, 8, 1], [3, 8, 1]], True), ([[3, 8, 1], [40, 2, 9, 17]], False)):
            st = g.stage(96, seqs=2)
            st.seqs_start(prompts)
            st.moe_stats()  # the prompts' batches counted so far
            st.seqs_run(steps)
            selected, groupings = st.moe_stats()
            assert groupings == SMALL.layers * steps
            if same:
                assert selected == 3 * groupings
            else:
                assert 3 * groupings <= selected <= 6 * groupings and selected > 3 * groupings
            assert st.moe_stats() == (0, 0)
            st.free()
    finally:
        g.free()
    assert dev.used == 0
