"""The decode step's attention values and Wo product in one launch
(launch_att_values_wo: the Wo workgroups request their rows at the launch's
start and wait for the values workgroups through device words) give the
oracle's bits, as the two launches do (internal/llm/model.go:575-596: the
attention output, its Q8_0 form, x += Wo·attn).

The launch takes a Q8_0 Wo of 3073..4096 columns (heads x head size) and
contexts of up to 1024 positions, so the models here have 32 heads of 128
(q_dim 4096) over a narrow residual: small enough for the oracle, the
shapes of config 3's and config 5's attention. Covered: the Llama, Qwen2
(QKV bias) and Qwen3 (QK-norm) attention paths with both values bodies
(contexts up to 256: four waves, Wo workgroups of 16 rows; longer: the
register-held values, Wo workgroups of 32 rows), decode positions on both
sides of 128, 256 and 512 (one to three chunks of values), many launches
of one stage (the launch counts carry over), two stages in turn (each its
own words), the layers-only forward, and eager launches (the profiler's
path)."""
import numpy as np
import pytest

from oracle.model import Config, Stage
from test_gpu_fused_stage import check_generation, coded_model, make_stage, same_bits

pytestmark = pytest.mark.gpu

BASE = dict(dim=512, hidden=512, layers=2, heads=32, kv_heads=8, head_dim=128, vocab=300, dtype="q8_0")


def fused_launches(dev, run):
    """The profile of run(): how many values-and-Wo launches it made, and
    whether any separate Wo product ran."""
    dev.profile_start()
    try:
        run()
    finally:
        prof = dev.profile_stop()
    return prof.get("att_values_wo", (0, 0.0))[0], prof.get("wo", (0, 0.0))[0]


@pytest.mark.parametrize("arch", ["llama", "qwen2", "qwen3"])
def test_values_and_wo_in_one_launch_every_logit(dev, arch):
    extra = {"qwen2": dict(qkv_bias=True, rope_theta=1e6, norm_eps=1e-6),
             "qwen3": dict(qk_norm=True, rope_theta=1e6, norm_eps=1e-6)}.get(arch, {})
    c = Config(seq_len=640, **BASE, **extra)
    m = coded_model(c, 21, 2e-5, 2e-4)
    # a prompt of 250 tokens (batched), then decode positions 250..529:
    # contexts from one chunk of 256 values to three
    prompt = [int(t) for t in np.random.default_rng(22).integers(0, c.vocab, 250)]
    check_generation(dev, m, prompt, 280, 640)


@pytest.mark.parametrize("arch", ["llama", "qwen2", "qwen3"])
def test_short_context_values_and_wo_every_logit(dev, arch):
    """Contexts up to 256 (the short values kernel's work in the launch,
    Wo workgroups of 16 rows): a 40-token prompt, then positions 40..169,
    across the values' 128-position chunk edge; the launches counted."""
    extra = {"qwen2": dict(qkv_bias=True, rope_theta=1e6, norm_eps=1e-6),
             "qwen3": dict(qk_norm=True, rope_theta=1e6, norm_eps=1e-6)}.get(arch, {})
    c = Config(seq_len=200, **{**BASE, "dim": 128}, **extra)  # Wo rows: a multiple of 16
    m = coded_model(c, 28, 2e-5, 2e-4)
    prompt = [int(t) for t in np.random.default_rng(29).integers(0, c.vocab, 40)]
    check_generation(dev, m, prompt, 130, 200)
    st, mats = make_stage(dev, m, 200)
    emb = dev.upload(m.embed.kind, m.embed.rows, m.embed.cols, m.embed.q, m.embed.scales)
    st.set_head(emb, emb, m.rms_final)
    st.generate_start(prompt)
    st.generate_run(len(prompt) - 1)
    n_fused, n_wo = fused_launches(dev, lambda: st.generate_run(3))
    assert n_fused == 3 * c.layers and n_wo == 0
    st.free()
    emb.free()
    for mt in mats:
        mt.free()
    assert dev.used == 0


def test_two_stages_in_turn_and_eager_launches(dev):
    c = Config(seq_len=320, **BASE)
    m1 = coded_model(c, 23, 2e-5, 2e-4)
    m2 = coded_model(c, 24, 2e-5, 2e-4)
    prompt = [int(t) for t in np.random.default_rng(25).integers(0, c.vocab, 260)]
    stages = []
    for m in (m1, m2):
        st, mats = make_stage(dev, m, 320)
        emb = dev.upload(m.embed.kind, m.embed.rows, m.embed.cols, m.embed.q, m.embed.scales)
        st.set_head(emb, emb, m.rms_final)
        stages.append((st, mats, emb))
    want = []
    for i, (st, _, _) in enumerate(stages):
        want.append(list(st.generate(prompt, 12)))
    # in turn, one position at a time, several times over
    for st, _, _ in stages:
        st.generate_start(prompt)
        st.generate_run(len(prompt) - 1)
    for _ in range(11):
        for st, _, _ in stages:
            st.generate_run(1)
    for i, (st, _, _) in enumerate(stages):
        st.generate_run(1)
        assert list(st.tokens(len(prompt), 12)) == want[i]
    # eager launches (each timed on its own) make the same tokens
    st = stages[0][0]
    st.generate_start(prompt)
    st.generate_run(len(prompt) - 1)
    n_fused, n_wo = fused_launches(dev, lambda: st.generate_run(12))
    assert n_fused == 12 * c.layers and n_wo == 0
    assert list(st.tokens(len(prompt), 12)) == want[0]
    for st, mats, emb in stages:
        st.free()
        emb.free()
        for mt in mats:
            mt.free()
    assert dev.used == 0


def test_layers_only_forward_matches_cpu(dev):
    """Stage.ForwardMany one token at a time (the layers-only replay) at
    positions past 256."""
    c = Config(seq_len=300, **BASE)
    m = coded_model(c, 26, 2e-5, 2e-4)
    cpu = Stage(m, 300)
    gpu, mats = make_stage(dev, m, 300)
    rng = np.random.default_rng(27)
    toks = [int(t) for t in rng.integers(0, c.vocab, 264)]
    a = np.stack([m.embed_token(t) for t in toks])
    gpu.forward(a[:258].copy(), 0)  # batched: the caches of positions 0..257
    for pos in range(258):
        cpu.forward(a[pos], pos)
    for pos in range(258, 264):
        x = cpu.forward(a[pos].copy(), pos)
        out = {}
        n_fused, n_wo = fused_launches(dev, lambda: out.update(y=gpu.forward(a[pos:pos + 1].copy(), pos)))
        assert n_fused == c.layers and n_wo == 0
        same_bits(out["y"][0], x, f"position {pos}")
    gpu.free()
    for mt in mats:
        mt.free()
    assert dev.used == 0
