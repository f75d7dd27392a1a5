"""Hugging Face models (internal/llm/hf.go ImportHF) on the GPU: synthetic
LLaMA, Qwen2 (query/key/value biases, tied classifier) and Qwen3 (per-head
q/k norms, a head width apart from dim/heads) models written as
safetensors shards, imported with quantization by rkhip.formats.import_hf,
moved to the GPU by stage_from_checkpoint and generating greedily there:
every logit of every step equals the CPU oracle's run of the same imported
model (the import itself is pinned against the models' float64 definition
on the CPU)."""
import json

import numpy as np
import pytest

from rkhip import formats as fm
from test_formats_hf import VARIANTS, hf_model, oracle_of
from test_gpu_fused_stage import oracle_generate, same_bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("quant", ["q8_0", "q4_m"])
@pytest.mark.parametrize("name", sorted(VARIANTS))
def test_hf_import_generates_like_cpu(dev, name, quant):
    hc, opts = VARIANTS[name]
    _, shards = hf_model(np.random.default_rng(len(name) + 7), hc, **opts)
    m = oracle_of(fm.import_hf(json.dumps(hc), shards), quant)
    ck = fm.import_hf(json.dumps(hc), shards, quant=quant)
    ctx, prompt, steps = 48, [2, 9, 31], 20
    print(f"hf import {name} {quant}: ctx {ctx}, {steps} steps", flush=True)
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
        same_bits(logits[k], want_l[k], f"{name} {quant} logits of step {k}")
    assert toks == want_t
    assert dev.used == 0
