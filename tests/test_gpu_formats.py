"""The reference's own checkpoint fixture (sdk/js/test/fixtures/
tiny-model.bin: internal/llm/testmodel.Checkpoint(1)) read and quantized by
rkhip.formats, moved to the GPU by stage_from_checkpoint, and generating
greedily there: every logit of every step equals the CPU oracle's run of
the same checkpoint, at each weight type the GPU layers take."""
import os

import numpy as np
import pytest

import rkhip
from rkhip import formats as fm
from oracle.model import Config, Model
from test_gpu_fused_stage import oracle_generate, same_bits

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load_fixture():
    with open(os.path.join(GOLDEN, "tiny-model.bin"), "rb") as f:
        return fm.read_checkpoint(f.read())


def oracle_model(ck, dtype):
    """The oracle's model of the same float32 checkpoint."""
    c = ck.config
    oc = Config(dim=c.dim, hidden=c.hidden_dim, layers=c.n_layers, heads=c.n_heads, kv_heads=c.n_kv_heads,
                vocab=c.vocab_size, seq_len=c.seq_len, dtype=dtype)
    raw = {"embed": ck.embed.f32, "rms_final": ck.head.rms_final, "wcls": ck.head.wcls.f32, "layers": []}
    for ly in ck.layers:
        raw["layers"].append({n: (getattr(ly, n).f32 if n.startswith("w") else getattr(ly, n))
                              for n in ("rms_att", "wq", "wk", "wv", "wo", "rms_ffn", "w1", "w2", "w3")})
    return Model(oc, raw)


@pytest.mark.parametrize("dtype", ["q8_0", "q4_m", "q4_0"])
def test_fixture_generates_like_cpu(dev, dtype):
    ck = load_fixture()
    m = oracle_model(ck, dtype)
    ck.quantize(dtype)
    ctx, prompt, steps = ck.config.seq_len, [1, 5, 9], 24
    want_t, want_l = oracle_generate(m, prompt, steps, ctx)
    cos, sin = m.rope(ctx)
    st, mats, embed, wcls = fm.stage_from_checkpoint(dev, ck, ctx, cos, sin)
    try:
        st.set_head(embed, wcls, ck.head.rms_final)
        st.generate_start(prompt)
        st.generate_run(len(prompt) - 1)
        logits = [st.generate_run(1, want_logits=True)[0] for _ in range(steps)]
        toks = list(st.tokens(len(prompt), steps))
    finally:
        st.free()
        for mt in mats:
            mt.free()
    for k in range(steps):
        same_bits(logits[k], want_l[k], f"{dtype} logits of step {k}")
    assert toks == want_t
    assert dev.used == 0
