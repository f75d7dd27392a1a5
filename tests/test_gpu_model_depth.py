"""Every logit at the benchmarked shapes, depths and positions against the
oracle (internal/llm/gpu_test.go:32-111 compares GPU stages with the CPU
path at every position; here at the configurations bench.py measures):

* config 3's 8B layer shape (head size 128, GQA 32/8) with a 530-token
  prompt through the batched prefill path, then 16 decode positions
  (530-545, past 512, where the decode attention reads each value slice in
  several chunks), with the full 128256-token classifier;
* all 32 layers at the 8B shape, a 4-token prompt and 4 decode steps;
* config 4's Qwen-7B Q4 layer (QKV bias, hidden 18944) with a 520-token
  prompt, then 8 decode positions.

The oracle runs its Q8 / Q4 products through its AVX2 block sums on the
host's threads (the same bits as its portable loops, tested on the CPU)."""
import os

import numpy as np
import pytest

from oracle import oracle
from oracle.model import Config, Layer
from test_gpu_fused_stage import check_generation, coded_model

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))

LLAMA8B = dict(dim=4096, hidden=14336, heads=32, kv_heads=8, vocab=128256, rope_theta=500000.0, dtype="q8_0")


def test_8b_shape_long_prompt_then_decode_every_logit(dev):
    c = Config(layers=2, seq_len=768, **LLAMA8B)
    m = coded_model(c, 7, 2e-5, 2e-4)  # config 3's scale range
    prompt = [int(t) for t in np.random.default_rng(30).integers(0, c.vocab, 530)]
    with oracle.matvec_threads(THREADS):
        check_generation(dev, m, prompt, 16, 768)


def test_8b_shape_all_32_layers_every_logit(dev):
    """32 layers of the 8B shape. Four weight sets are cycled over the
    layers (layer l takes set l mod 4; each layer still gets its own device
    copy and its own caches), and every layer has its own norm vectors, so
    every layer's arithmetic differs."""
    c = Config(layers=4, seq_len=64, **LLAMA8B)
    m = coded_model(c, 8, 2e-5, 2e-4)
    rng = np.random.default_rng(9)
    sets = m.layers
    m.layers = []
    for li in range(32):
        ly = Layer()
        for n in Layer.MATS:
            setattr(ly, n, getattr(sets[li % 4], n))
        ly.rms_att = rng.normal(1, 0.1, c.dim).astype(np.float32)
        ly.rms_ffn = rng.normal(1, 0.1, c.dim).astype(np.float32)
        m.layers.append(ly)
    m.c = Config(layers=32, seq_len=64, **LLAMA8B)
    with oracle.matvec_threads(THREADS):
        check_generation(dev, m, [11, 7000, 123, 99], 4, 64)


def test_qwen7b_q4_layer_long_prompt_every_logit(dev):
    c = Config(dim=3584, hidden=18944, layers=1, heads=28, kv_heads=4, vocab=152064, seq_len=576,
               rope_theta=1000000.0, qkv_bias=True, norm_eps=1e-6, dtype="q4_0")
    m = coded_model(c, 9, 2e-5, 2e-4)  # config 4's scale range
    prompt = [int(t) for t in np.random.default_rng(31).integers(0, c.vocab, 520)]
    with oracle.matvec_threads(THREADS):
        check_generation(dev, m, prompt, 8, 576)
