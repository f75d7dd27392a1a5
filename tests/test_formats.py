"""The reference's model formats on the host (rkhip.formats): llama2.c
checkpoints (internal/llm/model.go:702-800), model parts
(internal/llm/shard.go:166-290) and the weight quantizers Quantize uses
(internal/num/quant.go:24-126), against the reference's own fixture
(sdk/js/test/fixtures/tiny-model.bin) and the C oracle."""
import os

import numpy as np
import pytest

from oracle import oracle
from rkhip import formats as fm

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def fixture():
    with open(os.path.join(GOLDEN, "tiny-model.bin"), "rb") as f:
        return f.read()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def test_read_checkpoint_fixture():
    """testmodel.Checkpoint(1) (internal/llm/testmodel/testmodel.go:15-33):
    the header, every tensor in its slot (N(0,1) embedding and norm
    weights, N(0,0.2) matrices: a misplaced tensor shows in its spread), and
    Encode(ReadCheckpoint(b)) == b."""
    data = fixture()
    ck = fm.read_checkpoint(data)
    c = ck.config
    assert (c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.vocab_size, c.seq_len) == \
        (64, 160, 4, 4, 2, 50, 64)
    assert not c.shared_classifier and c.head_size() == 16 and c.kv_dim() == 32
    assert ck.encode() == data
    sd = lambda v: float(np.std(v))  # noqa: E731
    assert 0.9 < sd(ck.embed.f32) < 1.1 and 0.9 < sd(ck.head.rms_final) < 1.35
    assert 0.17 < sd(ck.head.wcls.f32) < 0.23
    for ly in ck.layers:
        assert 0.7 < sd(ly.rms_att) < 1.3 and 0.7 < sd(ly.rms_ffn) < 1.3
        for n, size in (("wq", 64 * 64), ("wk", 32 * 64), ("wv", 32 * 64), ("wo", 64 * 64), ("w1", 160 * 64),
                        ("w2", 64 * 160), ("w3", 160 * 64)):
            m = getattr(ly, n).f32
            assert m.size == size and 0.18 < sd(m) < 0.22, n


def test_read_checkpoint_errors():
    data = fixture()
    with pytest.raises(ValueError, match="checkpoint too short"):
        fm.read_checkpoint(data[:27])
    with pytest.raises(ValueError, match="checkpoint truncated"):
        fm.read_checkpoint(data[:-4])
    bad = bytearray(data)
    bad[12:16] = np.array([3], np.int32).tobytes()  # 3 heads do not divide dim 64
    with pytest.raises(ValueError, match="checkpoint: heads do not divide"):
        fm.read_checkpoint(bytes(bad))


def awkward(rng, n):
    v = rng.normal(0, 1, n).astype(np.float32)
    pick = rng.integers(0, 50, n)
    v[pick == 0] = rng.integers(1, 1 << 23, int(np.sum(pick == 0)), dtype=np.uint32).view(np.float32)
    v[pick == 1] = np.float32(-0.0)
    v[pick == 2] = np.float32(3e38)
    v[pick == 3] *= np.float32(1e-38)
    v[:32] = 0  # a zero block
    v[32:64] = rng.integers(1, 1 << 20, 32, dtype=np.uint32).view(np.float32)  # a block of denormals
    return v


def test_recip32_matches_oracle():
    rng = np.random.default_rng(1)
    x = np.concatenate([np.exp2(rng.uniform(-140, 127, 20000)).astype(np.float32),
                        rng.integers(1, 1 << 23, 2000, dtype=np.uint32).view(np.float32),
                        np.array([0, -0.0, np.inf, -np.inf, np.nan, 1, 3e38, 1e-45], np.float32)])
    x = np.concatenate([x, -x])
    got = fm.recip32(x)
    want = np.array([oracle.lib().rko_recip32(np.float32(v)) for v in x], np.float32)
    assert np.array_equal(bits(got), bits(want))


def test_quantizers_match_oracle():
    """QuantizeQ8 / QuantizeQ4 / ToBF16 restated in numpy give the oracle's
    bits: normal weights, denormals, zero blocks, huge values."""
    rng = np.random.default_rng(2)
    for w in (awkward(rng, 32 * 2000), rng.normal(0, 0.02, 32 * 3000).astype(np.float32),
              fm.read_checkpoint(fixture()).layers[0].w1.f32):
        q, s = fm.quantize_q8(w)
        oq, os_ = oracle.quantize8(w)
        assert np.array_equal(q, oq) and np.array_equal(bits(s), bits(os_))
        q, s = fm.quantize_q4(w)
        oq, os_ = oracle.quantize4(w)
        assert np.array_equal(q, oq) and np.array_equal(bits(s), bits(os_))
        assert np.array_equal(fm.to_bf16(w), oracle.to_bf16(w))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "q8_0", "q4_0", "q4_m"])
def test_model_parts_round_trip(dtype):
    """EncodeLayer / LoadLayer, EncodeHead / LoadHead and the embedding at
    every weight type: sizes are LayerBytes / EmbedBytes and the parts load
    back to the same values; a part of the wrong size is an error."""
    ck = fm.read_checkpoint(fixture())
    ck.quantize(dtype)
    c = ck.config
    for ly in ck.layers:
        b = fm.encode_layer(c, ly)
        assert len(b) == fm.layer_bytes(c)
        back = fm.load_layer(c, b)
        assert fm.encode_layer(c, back) == b
        with pytest.raises(ValueError, match="wrong size"):
            fm.load_layer(c, b + b"\0")
        with pytest.raises(ValueError, match="wrong size"):
            fm.load_layer(c, b[:-1])
    e = fm.append_matrix(ck.embed)
    assert len(e) == fm.embed_bytes(c)
    emb = fm.load_embed(c, e)
    hb = fm.encode_head(c, ck.head)
    head = fm.load_head(c, hb, emb)
    assert fm.encode_head(c, head) == hb
    assert fm.append_matrix(head.wcls) == fm.append_matrix(ck.head.wcls)


def test_quantize_types_follow_the_config():
    """model.go:96-113: q4_m keeps wv and w2 in q8_0, the embedding and
    classifier are q8_0 under q4_0 / q4_m."""
    ck = fm.read_checkpoint(fixture())
    ck.quantize("q4_m")
    ly = ck.layers[0]
    assert ly.wv.q8 is not None and ly.w2.q8 is not None
    assert all(getattr(ly, n).q4 is not None for n in ("wq", "wk", "wo", "w1", "w3"))
    assert ck.embed.q8 is not None and ck.head.wcls.q8 is not None
    with pytest.raises(ValueError):
        fm.read_checkpoint(fixture()).quantize("q5")
