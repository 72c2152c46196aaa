"""The synthetic checkpoint (lucciola_rs_amd/checkpoint.py): config.json +
safetensors in the reference's tensor names, read back by the reference's
loading rules and, independently, by the `safetensors` library (CPU only)."""
import json
import os

import numpy as np
import pytest
import torch

from lucciola_rs_amd.checkpoint import config_from_json, load_checkpoint, write_checkpoint
from lucciola_rs_amd.model import Qwen2Config, random_weights

TINY = Qwen2Config(vocab_size=1000, hidden_size=256, num_hidden_layers=3, num_attention_heads=4,
                   num_key_value_heads=2, intermediate_size=512, max_position_embeddings=4096,
                   eos_token_id=999, bos_token_id=998)


def same(a, b):
    return a.dtype == b.dtype and a.shape == b.shape and np.array_equal(a, b)


def check_same_weights(w, w2, tied=True):
    assert same(w["embed_tokens"], w2["embed_tokens"]) and same(w["final_norm"], w2["final_norm"])
    assert len(w["layers"]) == len(w2["layers"])
    for L, L2 in zip(w["layers"], w2["layers"]):
        assert L.keys() == L2.keys()
        for k in L:
            assert same(L[k], L2[k]), k
    assert ("lm_head" in w2) == (not tied)


@pytest.mark.parametrize("shards", [1, 3])
def test_round_trip(tmp_path, shards):
    w = random_weights(TINY, seed=5)
    files = write_checkpoint(str(tmp_path), TINY, w, shards=shards)
    assert len(files) == shards
    cfg, w2 = load_checkpoint(str(tmp_path))
    assert cfg == TINY
    check_same_weights(w, w2)


def test_untied_lm_head(tmp_path):
    cfg = Qwen2Config(**{**TINY.__dict__, "tie_word_embeddings": False})
    w = random_weights(cfg, seed=6)
    write_checkpoint(str(tmp_path), cfg, w)
    cfg2, w2 = load_checkpoint(str(tmp_path))
    assert not cfg2.tie_word_embeddings
    check_same_weights(w, w2, tied=False)
    assert same(w["lm_head"], w2["lm_head"])


def test_independent_reader_sees_hf_names_shapes_and_bytes(tmp_path):
    """The safetensors library parses the file; names, BF16 dtype, [out, in]
    shapes and values are those of the Hugging Face Qwen2 layout."""
    from safetensors import safe_open
    w = random_weights(TINY, seed=7)
    (path,) = write_checkpoint(str(tmp_path), TINY, w)
    H, I, d = TINY.hidden_size, TINY.intermediate_size, TINY.head_dim
    kv = TINY.num_key_value_heads * d
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    with safe_open(path, framework="pt") as f:
        names = set(f.keys())
        assert "lm_head.weight" not in names  # tied
        assert len(names) == 2 + TINY.num_hidden_layers * 12
        e = f.get_tensor("model.embed_tokens.weight")
        assert e.dtype == torch.bfloat16 and tuple(e.shape) == (TINY.vocab_size, H)
        assert np.array_equal(bits(e), w["embed_tokens"])
        shapes = {"self_attn.q_proj.weight": (H, H), "self_attn.k_proj.weight": (kv, H),
                  "self_attn.v_proj.weight": (kv, H), "self_attn.q_proj.bias": (H,),
                  "self_attn.k_proj.bias": (kv,), "self_attn.v_proj.bias": (kv,),
                  "self_attn.o_proj.weight": (H, H), "mlp.gate_proj.weight": (I, H),
                  "mlp.up_proj.weight": (I, H), "mlp.down_proj.weight": (H, I),
                  "input_layernorm.weight": (H,), "post_attention_layernorm.weight": (H,)}
        for n in range(TINY.num_hidden_layers):
            for k, shp in shapes.items():
                assert tuple(f.get_tensor(f"model.layers.{n}.{k}").shape) == shp, k
        L = w["layers"][1]
        assert np.array_equal(bits(f.get_tensor("model.layers.1.self_attn.k_proj.weight")),
                              L["qkv_proj"][H:H + kv])
        assert np.array_equal(bits(f.get_tensor("model.layers.1.self_attn.v_proj.bias")),
                              L["qkv_bias"][H + kv:])
        assert np.array_equal(bits(f.get_tensor("model.layers.1.mlp.up_proj.weight")),
                              L["gate_up_proj"][I:])
    with open(tmp_path / "config.json") as fh:
        c = json.load(fh)
    assert c["model_type"] == "qwen2" and c["num_key_value_heads"] == 2 and c["tie_word_embeddings"]


def test_missing_bias_gives_zeros(tmp_path):
    w = random_weights(TINY, seed=8)
    write_checkpoint(str(tmp_path), TINY, w, with_bias=False)
    _, w2 = load_checkpoint(str(tmp_path))
    bias_dim = TINY.hidden_size + 2 * TINY.num_key_value_heads * TINY.head_dim
    for L in w2["layers"]:
        assert L["qkv_bias"].shape == (bias_dim,) and not L["qkv_bias"].any()


def test_partial_bias_gives_zeros(tmp_path):
    """One of q/k/v bias missing: the whole fused bias is zeros (utils.rs:101-110)."""
    from lucciola_rs_amd.checkpoint import _hf_tensors, write_safetensors
    w = random_weights(TINY, seed=9)
    t = [(n, a) for n, a in _hf_tensors(TINY, w, True) if n != "model.layers.0.self_attn.k_proj.bias"]
    write_safetensors(str(tmp_path / "model.safetensors"), t)
    with open(tmp_path / "config.json", "w") as f:
        json.dump({**TINY.__dict__, "rope_scaling": None}, f)
    _, w2 = load_checkpoint(str(tmp_path))
    assert not w2["layers"][0]["qkv_bias"].any()
    assert same(w2["layers"][1]["qkv_bias"], w["layers"][1]["qkv_bias"])


def test_missing_tensor_and_missing_files(tmp_path):
    from lucciola_rs_amd.checkpoint import _hf_tensors, write_safetensors
    w = random_weights(TINY, seed=10)
    with open(tmp_path / "config.json", "w") as f:
        json.dump({**TINY.__dict__, "rope_scaling": None}, f)
    with pytest.raises(FileNotFoundError, match="No .safetensors"):
        load_checkpoint(str(tmp_path))
    t = [(n, a) for n, a in _hf_tensors(TINY, w, True) if n != "model.layers.2.mlp.up_proj.weight"]
    write_safetensors(str(tmp_path / "model.safetensors"), t)
    with pytest.raises(KeyError, match="Tensor model.layers.2.mlp.up_proj.weight not found"):
        load_checkpoint(str(tmp_path))


def test_first_file_in_sorted_order_wins(tmp_path):
    from lucciola_rs_amd.checkpoint import _hf_tensors, write_safetensors
    w = random_weights(TINY, seed=11)
    t = _hf_tensors(TINY, w, True)
    norm = np.full(TINY.hidden_size, 0x3f80, np.uint16)  # 1.0
    write_safetensors(str(tmp_path / "b.safetensors"), t)
    write_safetensors(str(tmp_path / "a.safetensors"), [("model.norm.weight", norm)])
    with open(tmp_path / "config.json", "w") as f:
        json.dump({**TINY.__dict__, "rope_scaling": None}, f)
    _, w2 = load_checkpoint(str(tmp_path))
    assert same(w2["final_norm"], norm)


def test_config_defaults_and_required_fields():
    d = {k: v for k, v in TINY.__dict__.items() if k not in ("rope_theta", "rms_norm_eps",
                                                            "rope_scaling_factor")}
    cfg = config_from_json(d)
    assert cfg.rope_theta == 1e6 and cfg.rms_norm_eps == 1e-6 and cfg.rope_scaling_factor is None
    cfg = config_from_json({**d, "rope_scaling": {"type": "linear", "factor": 4.0}})
    assert cfg.rope_scaling_factor == 4.0
    with pytest.raises(ValueError, match="vocab_size"):
        config_from_json({k: v for k, v in d.items() if k != "vocab_size"})


def test_oracle_loop_identical_from_checkpoint(tmp_path, orc):
    """The oracle's decoder built from a written-then-loaded checkpoint gives
    the same logits bit for bit as from the in-memory weights."""
    from oracle.model import OracleQwen2
    w = random_weights(TINY, seed=12, std=0.1)
    write_checkpoint(str(tmp_path), TINY, w, shards=2)
    cfg, w2 = load_checkpoint(str(tmp_path))
    a, b = OracleQwen2(TINY, w, 64), OracleQwen2(cfg, w2, 64)
    ids = [5, 17, 999, 0, 3]
    a.forward(ids, 0)
    b.forward(ids, 0)
    assert np.array_equal(a.logits(), b.logits())
    assert os.path.getsize(tmp_path / "config.json") > 0
