"""A model's layers on the GPU give the CPU oracle's bits (the reference's
TestGPUStagesMatchCPU, internal/llm/gpu_test.go:32-111): three architecture
variants (Qwen2 QKV bias; Qwen3 QK-norm with head_dim 32, theta 1e6, eps
1e-6; no GQA), each weight type the reference runs there (float32 "",
bf16, q8_0, q4_m, q4_0), a 70-token prompt (two submissions) and six decode
steps, every activation compared bitwise."""
import numpy as np
import pytest

from gpustage import GPUStage
from oracle.model import Config, Model, Stage, random_model

pytestmark = pytest.mark.gpu

CONFIGS = [
    Config(dim=64, hidden=128, layers=3, heads=4, kv_heads=2, vocab=50, seq_len=96, qkv_bias=True),
    Config(dim=64, hidden=96, layers=2, heads=4, kv_heads=2, vocab=50, seq_len=96, head_dim=32, qk_norm=True,
           rope_theta=1e6, norm_eps=1e-6),
    Config(dim=96, hidden=160, layers=2, heads=3, kv_heads=3, vocab=50, seq_len=96),
]


@pytest.mark.parametrize("ci", range(len(CONFIGS)))
@pytest.mark.parametrize("dtype", ["", "bf16", "q8_0", "q4_m", "q4_0"])
def test_gpu_stages_match_cpu(dev, ci, dtype):
    c = Config(**{**CONFIGS[ci].__dict__, "dtype": dtype})
    m = Model(c, random_model(c, 9))
    cpu = Stage(m, 80)
    gpu = GPUStage(dev, m, 80)
    prompt = [(i * 7 + 3) % c.vocab for i in range(70)]
    a = np.stack([m.embed_token(t) for t in prompt])
    b = a.copy()
    for pos in range(len(prompt)):
        a[pos] = cpu.forward(a[pos], pos)
    b = gpu.forward(b, 0, len(prompt))
    for pos in range(len(prompt)):
        assert np.array_equal(a[pos].view(np.uint32), b[pos].view(np.uint32)), f"prompt position {pos}"
    for i, tok in enumerate([16, 25, 36, 49, 7, 3]):
        pos = len(prompt) + i
        x = cpu.forward(m.embed_token(tok), pos)
        y = gpu.forward(m.embed_token(tok), pos, 1)[0]
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), f"decode position {pos}"
    gpu.close()
    assert dev.used == 0


def test_batch_spans_are_checked(dev):
    import rkhip

    a = dev.arena(64, 64)
    b = a.begin()
    assert b.copy(0, 60, 8) == rkhip.RK_ERR_ARGS  # leaves the arena
    assert b.residual(0, 8, 8, False) == rkhip.RK_ERR_ARGS  # latched: later ops do nothing
    with pytest.raises(rkhip.RKError) as e:
        b.submit()
    assert e.value.code == rkhip.RK_ERR_ARGS
    b = a.begin()
    assert b.matvecs([], [], 0) == 0
    b.submit()
    a.free()
    assert dev.used == 0
