"""Independent sequences (rk_stage_seqs_*) on dense layers: the
coordinator's concurrent generations (internal/llm/generate.go:415-522)
decoded side by side, each with its own position and caches, on the layer
types the MoE stage tests do not reach:
* QKV bias (Qwen2, model.go:541-549): the batched products' QKV epilogue
  writing each sequence's caches through its position;
* no QK-norm (Llama), with and without GQA: the scores and values launches
  with a per-sequence position and cache offset;
* a QK-norm head wider than the fused norm-and-scores launch takes (head
  size 320): the separate QK-norm launch;
* dense SwiGLU feed-forwards, Q8 and Q4 weights.
Prompts of different lengths. Every logit and token of every sequence is
the oracle's (internal/llm/model.go:522-673, sample.go:45-53), and each
sequence's tokens equal the same sequence's on a one-sequence stage."""
import numpy as np
import pytest

import rkhip
from oracle.model import Config
from test_gpu_fused_stage import coded_model, gpu_generate, oracle_generate, same_bits, upload_layers

pytestmark = pytest.mark.gpu

CASES = {
    "qwen2_bias": Config(dim=64, hidden=128, layers=2, heads=4, kv_heads=2, vocab=50, seq_len=96, qkv_bias=True,
                         rope_theta=1e6, norm_eps=1e-6, dtype="q8_0"),
    "llama_gqa": Config(dim=128, hidden=192, layers=2, heads=8, kv_heads=2, vocab=50, seq_len=96, dtype="q8_0"),
    "llama_mha": Config(dim=96, hidden=160, layers=2, heads=3, kv_heads=3, vocab=50, seq_len=96, dtype="q8_0"),
    "llama_q4": Config(dim=128, hidden=256, layers=2, heads=4, kv_heads=2, vocab=50, seq_len=96, dtype="q4_0"),
    "qknorm_hs320": Config(dim=64, hidden=96, layers=2, heads=2, kv_heads=1, vocab=50, seq_len=96, head_dim=320,
                           qk_norm=True, rope_theta=1e6, norm_eps=1e-6, dtype="q8_0"),
}


def seqs_generate(dev, m, prompts, steps, ctx):
    """Every sequence through one stage of len(prompts) sequences: the
    logits [steps][seqs][vocab] and each sequence's tokens."""
    c = m.c
    layers, mats = upload_layers(dev, m)
    emb = dev.upload(m.embed.kind, m.embed.rows, m.embed.cols, m.embed.q, m.embed.scales)
    cos, sin = m.rope(ctx)
    st = rkhip.Stage(dev, c.dim, c.hidden, c.heads, c.kv_heads, ctx, layers, cos, sin, head_dim=c.head_dim,
                     norm_eps=float(c.eps()), qkv_bias=c.qkv_bias, qk_norm=c.qk_norm, seqs=len(prompts))
    try:
        st.set_head(emb, emb, m.rms_final)
        st.seqs_start(prompts)
        lg = st.seqs_run(steps, want_logits=True)
        toks = [list(st.seqs_tokens(z, len(p), steps)) for z, p in enumerate(prompts)]
    finally:
        st.free()
        emb.free()
        for mt in mats:
            mt.free()
    return lg, toks


@pytest.mark.parametrize("name", sorted(CASES))
def test_dense_sequences_match_each_alone(dev, name):
    c = CASES[name]
    m = coded_model(c, seed=7, scale_lo=1e-3, scale_hi=1e-2)
    rng = np.random.default_rng(3)
    prompts = [[int(t) for t in rng.integers(0, c.vocab, n)] for n in (1, 2, 9, 30, 17)]
    steps, ctx = 8, 64
    lg, toks = seqs_generate(dev, m, prompts, steps, ctx)
    for z, p in enumerate(prompts):
        want_t, want_l = oracle_generate(m, p, steps, ctx)
        for k in range(steps):
            same_bits(lg[k, z], want_l[k], f"{name}: sequence {z} (prompt {len(p)}), step {k}")
        assert toks[z] == want_t, f"{name}: sequence {z} tokens"
        alone, _, _ = gpu_generate(dev, m, p, steps, ctx)
        assert alone == toks[z], f"{name}: sequence {z} alone"
    assert dev.used == 0
