"""Hugging Face import (internal/llm/hf.go) on the CPU: safetensors files
written here from synthetic weights, read by rkhip.formats.import_hf.

Pins: f16_to_f32 against numpy's half conversion over every non-NaN bit
pattern (NaN payloads by their closed form); permute_rows against its
index rule; config.json's mapping against the reference's defaults and
errors (hf.go:253-307); and the import as a whole against a float64
forward written from the Hugging Face models' own definition (rotate-half
rotary embedding on the unpermuted rows, gate/up/down MLP, biases, per-head
q/k norms, grouped heads): the oracle engine running the imported model
gives the same logits to float32 accuracy, and a wrong row permutation,
a swapped projection or a dropped bias does not."""
import json

import numpy as np
import pytest

from rkhip import formats as fm
from oracle.model import Config as OConfig, Model, Stage

def st_bytes(tensors, meta=None):
    """A safetensors file: name -> (dtype, shape, little-endian bytes)."""
    hdr, off, blobs = {}, 0, []
    if meta is not None:
        hdr["__metadata__"] = meta
    for name, (dt, shape, b) in tensors.items():
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    return np.array([len(h)], "<u8").tobytes() + h + b"".join(blobs)


def f32t(a, shape):
    return ("F32", shape, np.ascontiguousarray(a, "<f4").tobytes())


def bf16t(a, shape):
    return ("BF16", shape, np.ascontiguousarray(fm.to_bf16(a), "<u2").tobytes())


def f16t(a, shape):
    return ("F16", shape, np.ascontiguousarray(np.asarray(a, np.float16).view(np.uint16), "<u2").tobytes())


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# --- pieces ------------------------------------------------------------------

def test_f16_to_f32_every_pattern():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = fm.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(bits(got)[~nan], bits(ref)[~nan])
    # NaNs: sign, all-ones exponent, the 10 payload bits shifted up 13
    hn = h[nan].astype(np.uint32)
    want = ((hn >> 15) << 31) | 0x7F800000 | ((hn & 0x3FF) << 13)
    assert np.array_equal(bits(got)[nan], want)
    assert bits(fm.f16_to_f32([0x0001]))[0] == 0x33800000  # 2^-24
    assert bits(fm.f16_to_f32([0x8000]))[0] == 0x80000000


def test_permute_rows_index_rule():
    head, n, heads = 8, 3, 2
    w = np.arange(heads * head * n, dtype=np.float32)
    got = fm.permute_rows(w, heads * head, head).reshape(heads * head, n)
    src = w.reshape(heads * head, n)
    for hb in range(heads):
        for j in range(head // 2):
            assert np.array_equal(got[hb * head + 2 * j], src[hb * head + j])
            assert np.array_equal(got[hb * head + 2 * j + 1], src[hb * head + j + head // 2])
    v = np.arange(16, dtype=np.float32)
    assert fm.permute_vec(v, 8).tolist() == [0, 4, 1, 5, 2, 6, 3, 7, 8, 12, 9, 13, 10, 14, 11, 15]


def test_read_safetensors_tensors_and_errors():
    rng = np.random.default_rng(1)
    a = rng.normal(0, 1, 6).astype(np.float32)
    b = st_bytes({"x": f32t(a, (2, 3)), "y": bf16t(a[:4], (4,))}, meta={"format": "pt"})
    ts = {}
    fm.read_safetensors(b, ts)
    assert sorted(ts) == ["x", "y"]
    raw, size = ts["x"].raw("x", 6)
    assert size == 4 and np.array_equal(np.frombuffer(raw, "<f4"), a)
    with pytest.raises(ValueError, match=r"tensor x: shape \[2, 3\], want 5 elements"):
        ts["x"].raw("x", 5)
    with pytest.raises(ValueError, match="safetensors: tensor x in two files"):
        fm.read_safetensors(b, ts)
    with pytest.raises(ValueError, match="safetensors: header of"):
        fm.read_safetensors(np.array([1 << 40], "<u8").tobytes() + b"{}", {})
    bad = st_bytes({"x": ("F32", (4,), b"\0" * 16)})
    with pytest.raises(ValueError, match="safetensors tensor x: data outside the file"):
        fm.read_safetensors(bad[:-4], {})
    ts = {}
    fm.read_safetensors(st_bytes({"z": ("I64", (2,), b"\0" * 16)}), ts)
    with pytest.raises(ValueError, match="tensor z: type I64 not supported"):
        ts["z"].raw("z", 2)


def test_read_safetensors_from_disk(tmp_path):
    a = np.arange(8, dtype=np.float32)
    p = tmp_path / "m.safetensors"
    p.write_bytes(st_bytes({"w": f32t(a, (8,))}))
    ts = {}
    fm.read_safetensors(str(p), ts)
    raw, _ = ts["w"].raw("w", 8)
    assert np.array_equal(np.frombuffer(raw, "<f4"), a)


# --- config.json ---------------------------------------------------------------

def llama_cfg(**kw):
    hc = {"model_type": "llama", "hidden_size": 64, "intermediate_size": 96, "num_hidden_layers": 2,
          "num_attention_heads": 4, "num_key_value_heads": 2, "vocab_size": 50, "max_position_embeddings": 64,
          "hidden_act": "silu"}
    hc.update(kw)
    return {k: v for k, v in hc.items() if v is not None}


def weights_of(*names, embed="F32"):
    ts = {n: fm.STTensor("F32", [1], (0, 4)) for n in names}
    ts["model.embed_tokens.weight"] = fm.STTensor(embed, [1], (0, 4))
    return ts


def test_hf_config_defaults():
    c = fm.hf_config_of(llama_cfg(num_key_value_heads=None), weights_of("lm_head.weight"))
    assert (c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.vocab_size, c.seq_len) == \
        (64, 96, 2, 4, 4, 50, 64)
    assert c.rope_theta == 10000 and c.norm_eps == 1e-6 and c.head_dim == 0
    assert not c.shared_classifier and not c.qkv_bias and not c.qk_norm and c.dtype == "f32"
    # no lm_head: shared; tied: shared even with one
    assert fm.hf_config_of(llama_cfg(), weights_of()).shared_classifier
    assert fm.hf_config_of(llama_cfg(tie_word_embeddings=True), weights_of("lm_head.weight")).shared_classifier
    # head_dim only when it differs from dim / heads
    assert fm.hf_config_of(llama_cfg(head_dim=16), weights_of()).head_dim == 0
    assert fm.hf_config_of(llama_cfg(head_dim=32), weights_of()).head_dim == 32
    c = fm.hf_config_of(llama_cfg(model_type="qwen3", rope_theta=1e6, rms_norm_eps=1e-5),
                        weights_of("model.layers.0.self_attn.q_proj.bias", "model.layers.0.self_attn.q_norm.weight",
                                   embed="BF16"))
    assert c.qkv_bias and c.qk_norm and c.dtype == "bf16" and c.rope_theta == 1e6 and c.norm_eps == 1e-5


def test_hf_config_sliding_window():
    w = weights_of()
    assert fm.hf_config_of(llama_cfg(sliding_window=32), w).seq_len == 32
    assert fm.hf_config_of(llama_cfg(sliding_window=32, use_sliding_window=False), w).seq_len == 64
    assert fm.hf_config_of(llama_cfg(sliding_window=128), w).seq_len == 64
    assert fm.hf_config_of(llama_cfg(sliding_window=0), w).seq_len == 64


@pytest.mark.parametrize("kw,msg", [
    ({"model_type": "gemma"}, 'model type "gemma" is not supported'),
    ({"hidden_act": "gelu"}, 'activation "gelu" is not supported'),
    ({"rope_scaling": {"type": "linear", "factor": 2.0}}, "rope scaling .* is not supported"),
    ({"num_attention_heads": 5}, "heads do not divide the model dimension evenly"),
    ({"hidden_size": 0}, "non-positive dimension"),
])
def test_hf_config_errors(kw, msg):
    with pytest.raises(ValueError, match=msg):
        fm.hf_config_of(llama_cfg(**kw), weights_of())


def test_hf_config_refuses_output_bias():
    with pytest.raises(ValueError, match="output projection biases are not supported"):
        fm.hf_config_of(llama_cfg(), weights_of("model.layers.0.self_attn.o_proj.bias"))


# --- whole models ---------------------------------------------------------------

def hf_model(rng, hc, bias=False, qk_norm=False, tied=False, kinds="F32", wscale=0.15):
    """Random weights in Hugging Face names and shapes (out, in), split over
    two safetensors shards. Returns (float32 weights by name, [shard bytes])."""
    d, h, nl = hc["hidden_size"], hc["intermediate_size"], hc["num_hidden_layers"]
    nh, nkv, v = hc["num_attention_heads"], hc["num_key_value_heads"], hc["vocab_size"]
    hs = hc.get("head_dim") or d // nh
    W = {}

    def r(name, shape, s):
        W[name] = (rng.normal(0, 1, int(np.prod(shape))) * s).astype(np.float32).reshape(shape)

    r("model.embed_tokens.weight", (v, d), 1.0)
    r("model.norm.weight", (d,), 1.0)
    W["model.norm.weight"] += 1
    if not tied:
        r("lm_head.weight", (v, d), wscale)
    for i in range(nl):
        p = f"model.layers.{i}."
        r(p + "input_layernorm.weight", (d,), 0.3)
        r(p + "post_attention_layernorm.weight", (d,), 0.3)
        W[p + "input_layernorm.weight"] += 1
        W[p + "post_attention_layernorm.weight"] += 1
        r(p + "self_attn.q_proj.weight", (nh * hs, d), wscale)
        r(p + "self_attn.k_proj.weight", (nkv * hs, d), wscale)
        r(p + "self_attn.v_proj.weight", (nkv * hs, d), wscale)
        r(p + "self_attn.o_proj.weight", (d, nh * hs), wscale)
        r(p + "mlp.gate_proj.weight", (h, d), wscale)
        r(p + "mlp.up_proj.weight", (h, d), wscale)
        r(p + "mlp.down_proj.weight", (d, h), wscale)
        if bias:
            r(p + "self_attn.q_proj.bias", (nh * hs,), 0.5)
            r(p + "self_attn.k_proj.bias", (nkv * hs,), 0.5)
            r(p + "self_attn.v_proj.bias", (nkv * hs,), 0.5)
        if qk_norm:
            r(p + "self_attn.q_norm.weight", (hs,), 0.3)
            r(p + "self_attn.k_norm.weight", (hs,), 0.3)
            W[p + "self_attn.q_norm.weight"] += 1
            W[p + "self_attn.k_norm.weight"] += 1
    enc = {"F32": f32t, "BF16": bf16t, "F16": f16t}[kinds]
    names = sorted(W)
    shards = [{n: enc(W[n], W[n].shape) for n in names[k::2]} for k in range(2)]
    # what the file holds, as float32
    if kinds == "BF16":
        W = {n: (fm.to_bf16(a).astype(np.uint32) << 16).view(np.float32).reshape(a.shape) for n, a in W.items()}
    elif kinds == "F16":
        W = {n: a.astype(np.float16).astype(np.float32) for n, a in W.items()}
    return W, [st_bytes(s) for s in shards]


def hf_forward(W, hc, tokens):
    """The Hugging Face LLaMA / Qwen2 / Qwen3 forward in float64 from the
    models' definition: rotate-half rotary embedding over the original
    rows (dimension j turns with j + head/2 at frequency theta^(-2j/head)),
    causal attention over grouped key/value heads, SiLU-gated MLP. Returns
    every position's logits."""
    d, nl = hc["hidden_size"], hc["num_hidden_layers"]
    nh, nkv = hc["num_attention_heads"], hc["num_key_value_heads"]
    hs = hc.get("head_dim") or d // nh
    eps = hc.get("rms_norm_eps") or 1e-6
    theta = hc.get("rope_theta") or 10000.0
    g = {n: a.astype(np.float64) for n, a in W.items()}
    lm = g.get("lm_head.weight", g["model.embed_tokens.weight"])
    if hc.get("tie_word_embeddings"):
        lm = g["model.embed_tokens.weight"]

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w

    half = hs // 2
    inv = theta ** (-2.0 * np.arange(half) / hs)

    def rope(x, pos):  # x (heads, hs)
        a = pos * inv
        c, s = np.cos(a), np.sin(a)
        x1, x2 = x[:, :half], x[:, half:]
        return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=1)

    keys = [[] for _ in range(nl)]
    vals = [[] for _ in range(nl)]
    out = []
    for pos, tok in enumerate(tokens):
        x = g["model.embed_tokens.weight"][tok].copy()
        for i in range(nl):
            p = f"model.layers.{i}."
            xn = rms(x, g[p + "input_layernorm.weight"])
            q = g[p + "self_attn.q_proj.weight"] @ xn
            k = g[p + "self_attn.k_proj.weight"] @ xn
            v = g[p + "self_attn.v_proj.weight"] @ xn
            if p + "self_attn.q_proj.bias" in g:
                q = q + g[p + "self_attn.q_proj.bias"]
                k = k + g[p + "self_attn.k_proj.bias"]
                v = v + g[p + "self_attn.v_proj.bias"]
            q, k, v = q.reshape(nh, hs), k.reshape(nkv, hs), v.reshape(nkv, hs)
            if p + "self_attn.q_norm.weight" in g:
                q = rms(q, g[p + "self_attn.q_norm.weight"])
                k = rms(k, g[p + "self_attn.k_norm.weight"])
            q, k = rope(q, pos), rope(k, pos)
            keys[i].append(k)
            vals[i].append(v)
            K, V = np.stack(keys[i]), np.stack(vals[i])  # (t, nkv, hs)
            att = np.empty((nh, hs))
            for hh in range(nh):
                kv = hh // (nh // nkv)
                sc = K[:, kv, :] @ q[hh] / np.sqrt(hs)
                w = np.exp(sc - sc.max())
                att[hh] = (w / w.sum()) @ V[:, kv, :]
            x = x + g[p + "self_attn.o_proj.weight"] @ att.ravel()
            xn = rms(x, g[p + "post_attention_layernorm.weight"])
            a = g[p + "mlp.gate_proj.weight"] @ xn
            x = x + g[p + "mlp.down_proj.weight"] @ ((a / (1 + np.exp(-a))) * (g[p + "mlp.up_proj.weight"] @ xn))
        out.append(lm @ rms(x, g["model.norm.weight"]))
    return out


def oracle_of(ck, dtype="f32"):
    """The oracle engine's model of an imported float checkpoint."""
    c = ck.config
    oc = OConfig(dim=c.dim, hidden=c.hidden_dim, layers=c.n_layers, heads=c.n_heads, kv_heads=c.n_kv_heads,
                 vocab=c.vocab_size, seq_len=c.seq_len, head_dim=c.head_dim, rope_theta=c.rope_theta,
                 norm_eps=c.norm_eps, qkv_bias=c.qkv_bias, qk_norm=c.qk_norm, dtype=dtype)
    raw = {"embed": ck.embed.floats(), "rms_final": ck.head.rms_final, "layers": []}
    if not c.shared_classifier:
        raw["wcls"] = ck.head.wcls.floats()
    for ly in ck.layers:
        L = {n: getattr(ly, n).floats() for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3")}
        for n in ("rms_att", "rms_ffn", "bq", "bk", "bv", "q_norm", "k_norm"):
            if getattr(ly, n) is not None:
                L[n] = getattr(ly, n)
        raw["layers"].append(L)
    return Model(oc, raw)


def oracle_logits(m, tokens):
    st = Stage(m, len(tokens))
    out = []
    for pos, tok in enumerate(tokens):
        x = st.forward(m.embed_token(tok), pos)
        out.append(m.logits(x).astype(np.float64))
    return out


VARIANTS = {
    "llama": (llama_cfg(rope_theta=50.0, rms_norm_eps=1e-5), {}),
    "qwen2-bias": (llama_cfg(model_type="qwen2", rope_theta=50.0, tie_word_embeddings=True), {"bias": True,
                                                                                               "tied": True}),
    "qwen3-qknorm": (llama_cfg(model_type="qwen3", rope_theta=80.0, head_dim=32), {"qk_norm": True}),
}


@pytest.mark.parametrize("name", sorted(VARIANTS))
def test_import_matches_hf_definition(name):
    hc, opts = VARIANTS[name]
    rng = np.random.default_rng(len(name))
    W, shards = hf_model(rng, hc, **opts)
    ck = fm.import_hf(json.dumps(hc).encode(), shards[::-1])
    c = ck.config
    assert c.dtype == "f32" and c.qkv_bias == opts.get("bias", False) and c.qk_norm == opts.get("qk_norm", False)
    tokens = [3, 17, 42, 8, 29, 11]
    want = hf_forward(W, hc, tokens)
    got = oracle_logits(oracle_of(ck), tokens)
    for pos in range(len(tokens)):
        scale = np.max(np.abs(want[pos]))
        np.testing.assert_allclose(got[pos], want[pos], rtol=0, atol=2e-5 * scale + 1e-6,
                                   err_msg=f"{name} position {pos}")


def _inverse_permutation(ck):
    """Replace the stored query/key rows by the inverse permutation of the
    Hugging Face rows (what a swapped index rule would store)."""
    hs = ck.config.head_size()
    for ly in ck.layers:
        for n, rows in (("wq", ck.config.q_dim()), ("wk", ck.config.kv_dim())):
            fr = getattr(ly, n).f32.reshape(rows, -1)
            back, inv = np.empty_like(fr), np.empty_like(fr)
            for hb in range(0, rows, hs):
                for j in range(hs // 2):
                    back[hb + j] = fr[hb + 2 * j]
                    back[hb + j + hs // 2] = fr[hb + 2 * j + 1]
            for hb in range(0, rows, hs):
                for j in range(hs // 2):
                    inv[hb + j] = back[hb + 2 * j]
                    inv[hb + j + hs // 2] = back[hb + 2 * j + 1]
            setattr(ly, n, fm.Matrix(f32=inv.ravel()))


def _swap_gate_up(ck):
    for ly in ck.layers:
        ly.w1, ly.w3 = ly.w3, ly.w1


def _drop_bias(ck):
    for ly in ck.layers:
        ly.bk = np.zeros_like(ly.bk)


def _unpermuted_norm(ck):
    hs = ck.config.head_size()
    for ly in ck.layers:
        back = np.empty_like(ly.q_norm)
        back[:hs // 2], back[hs // 2:] = ly.q_norm[0::2], ly.q_norm[1::2]
        ly.q_norm = back


@pytest.mark.parametrize("variant,plant", [("llama", _inverse_permutation), ("llama", _swap_gate_up),
                                           ("qwen2-bias", _drop_bias), ("qwen3-qknorm", _unpermuted_norm)])
def test_planted_mistakes_are_caught(variant, plant):
    """The float64 check tells a correct import from one with a mistake
    planted in the imported parts (on the CPU)."""
    hc, opts = VARIANTS[variant]
    W, shards = hf_model(np.random.default_rng(5), hc, **opts)
    ck = fm.import_hf(json.dumps(hc).encode(), shards)
    plant(ck)
    tokens = [3, 17, 42, 8]
    want = hf_forward(W, hc, tokens)
    got = oracle_logits(oracle_of(ck), tokens)
    assert np.max(np.abs(got[-1] - want[-1])) > 1e-2 * np.max(np.abs(want[-1]))


@pytest.mark.parametrize("kinds", ["BF16", "F16"])
def test_half_weights_import(kinds):
    """bfloat16 files keep their bits for a bfloat16 model (hf.go:203-216);
    float16 files convert exactly; both follow the same forward."""
    hc, opts = VARIANTS["qwen2-bias"]
    W, shards = hf_model(np.random.default_rng(11), hc, kinds=kinds, **opts)
    ck = fm.import_hf(json.dumps(hc).encode(), shards)
    assert ck.config.dtype == ("bf16" if kinds == "BF16" else "f32")
    if kinds == "BF16":
        assert ck.embed.bf16 is not None and ck.layers[0].wv.bf16 is not None
        assert np.array_equal(ck.layers[1].w2.bf16, fm.to_bf16(W["model.layers.1.mlp.down_proj.weight"]).ravel())
    tokens = [1, 2, 3, 4]
    want = hf_forward(W, hc, tokens)
    got = oracle_logits(oracle_of(ck, ck.config.dtype), tokens)
    for pos in range(len(tokens)):
        np.testing.assert_allclose(got[pos], want[pos], rtol=0, atol=3e-5 * np.max(np.abs(want[pos])) + 1e-6)


@pytest.mark.parametrize("quant", ["q8_0", "q4_m", "bf16"])
def test_import_quant_is_quantize_of_permuted_floats(quant):
    """hf.go:325-330, 206-232, 420-428: quant stores each matrix as the
    config's type for it, the query and key rows permuted first; the parts
    equal Checkpoint.quantize of the float import, and round-trip through
    encode_layer / load_layer."""
    hc, opts = VARIANTS["qwen3-qknorm"]
    W, shards = hf_model(np.random.default_rng(2), hc, **opts)
    q = fm.import_hf(json.dumps(hc), shards, quant=quant)
    f = fm.import_hf(json.dumps(hc), shards)
    f.quantize(quant)
    assert q.config == f.config
    for a, b in zip(q.layers, f.layers):
        for n, is_mat, _, _, _ in fm.tensors(q.config):
            x, y = getattr(a, n), getattr(b, n)
            if is_mat:
                assert fm.append_matrix(x) == fm.append_matrix(y), n
            else:
                assert np.array_equal(bits(x), bits(y)), n
        part = fm.encode_layer(q.config, a)
        assert len(part) == fm.layer_bytes(q.config)
        assert fm.encode_layer(q.config, fm.load_layer(q.config, part)) == part
    assert fm.append_matrix(q.embed) == fm.append_matrix(f.embed)
    assert fm.encode_head(q.config, q.head) == fm.encode_head(f.config, f.head)


def test_import_errors():
    hc, opts = VARIANTS["llama"]
    W, shards = hf_model(np.random.default_rng(4), hc, **opts)
    with pytest.raises(ValueError, match="config.json"):
        fm.import_hf(b"{not json", shards)
    with pytest.raises(ValueError, match="tensor model.layers.1.mlp.up_proj.weight missing"):
        ts = {}
        fm.read_safetensors(shards[0], ts)
        fm.read_safetensors(shards[1], ts)
        hm = fm.HFModel(fm.hf_config_of(hc, ts), {k: v for k, v in ts.items() if "1.mlp.up_proj" not in k})
        hm.layer(1)
    bad = dict(hc, intermediate_size=97)
    with pytest.raises(ValueError, match="mlp.gate_proj.weight: shape"):
        fm.import_hf(json.dumps(bad), shards)
    with pytest.raises(ValueError, match="q8_0 needs widths that are multiples of 32"):
        fm.import_hf(json.dumps(dict(hc, intermediate_size=40)), shards, quant="q8_0")
    with pytest.raises(ValueError, match='unknown weight type "q9"'):
        fm.import_hf(json.dumps(hc), shards, quant="q9")
