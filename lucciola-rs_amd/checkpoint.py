"""The on-disk checkpoint the reference loads: `config.json` plus one or more
`*.safetensors` files with Hugging Face Qwen2 tensor names, bf16.

Writer: `write_checkpoint(dir, cfg, weights)` stores a weight set (the fused
layout of lucciola_rs_amd.model.random_weights) split back into the per-matrix
tensors the reference's loader looks up by name (src/models.rs:91-155):
  model.embed_tokens.weight                      [vocab, hidden]
  model.layers.N.input_layernorm.weight          [hidden]
  model.layers.N.self_attn.{q,k,v}_proj.weight   [Hq*d | Hkv*d | Hkv*d, hidden]
  model.layers.N.self_attn.{q,k,v}_proj.bias     (optional)
  model.layers.N.self_attn.o_proj.weight         [hidden, hidden]
  model.layers.N.post_attention_layernorm.weight [hidden]
  model.layers.N.mlp.{gate,up}_proj.weight       [inter, hidden]
  model.layers.N.mlp.down_proj.weight            [hidden, inter]
  model.norm.weight                              [hidden]
  lm_head.weight                                 (only when not tied)
The safetensors container (8-byte little-endian header length, JSON header of
dtype / shape / data_offsets, then the raw bytes) is written here directly.

Loader: `load_checkpoint(dir)` follows the reference's rules:
  * every `*.safetensors` file of the directory, in sorted path order
    (models.rs:60-70); a name is taken from the first file that has it;
  * tensor bytes are read as bf16 whatever the header's dtype says
    (utils.rs:20-34, which does no dtype check);
  * q|k|v and gate|up are concatenated (utils.rs:36-67); if any of the three
    q/k/v biases is missing, the bias is zeros of Hq*d + 2*Hkv*d
    (utils.rs:68-126);
  * lm_head is the embedding when tie_word_embeddings (models.rs:92-96);
  * a missing tensor raises "Tensor <name> not found" (utils.rs:34, 58).
config.json carries the fields of src/config.rs:3-37; rope_theta defaults to
1e6 and rms_norm_eps to 1e-6 when absent.
"""
from __future__ import annotations

import glob
import json
import os
import struct

import numpy as np

from .model import Qwen2Config

_REQUIRED = ("vocab_size", "max_position_embeddings", "num_hidden_layers", "hidden_size",
             "num_attention_heads", "num_key_value_heads", "intermediate_size", "eos_token_id",
             "bos_token_id", "tie_word_embeddings")


def config_to_json(cfg: Qwen2Config) -> dict:
    d = {k: getattr(cfg, k) for k in _REQUIRED}
    d.update(model_type="qwen2", rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_norm_eps,
             torch_dtype="bfloat16",
             rope_scaling=None if cfg.rope_scaling_factor is None
             else {"type": "linear", "factor": cfg.rope_scaling_factor})
    return d


def config_from_json(d: dict) -> Qwen2Config:
    """src/config.rs:3-37: the listed fields are required; rope_theta and
    rms_norm_eps have defaults; rope_scaling is optional."""
    missing = [k for k in _REQUIRED if k not in d]
    if missing:
        raise ValueError(f"config.json: missing field(s) {', '.join(missing)}")
    rs = d.get("rope_scaling")
    return Qwen2Config(**{k: d[k] for k in _REQUIRED},
                       rope_theta=float(d.get("rope_theta", 1e6)),
                       rms_norm_eps=float(d.get("rms_norm_eps", 1e-6)),
                       rope_scaling_factor=None if rs is None else float(rs["factor"]))


def _hf_tensors(cfg: Qwen2Config, w: dict, with_bias: bool) -> list[tuple[str, np.ndarray]]:
    H, I = cfg.hidden_size, cfg.intermediate_size
    kv = cfg.num_key_value_heads * cfg.head_dim
    out = [("model.embed_tokens.weight", w["embed_tokens"])]
    for n, L in enumerate(w["layers"]):
        p = f"model.layers.{n}."
        qkv, b = L["qkv_proj"], L["qkv_bias"]
        out += [(p + "input_layernorm.weight", L["input_layernorm"]),
                (p + "self_attn.q_proj.weight", qkv[:H]),
                (p + "self_attn.k_proj.weight", qkv[H:H + kv]),
                (p + "self_attn.v_proj.weight", qkv[H + kv:])]
        if with_bias:
            out += [(p + "self_attn.q_proj.bias", b[:H]), (p + "self_attn.k_proj.bias", b[H:H + kv]),
                    (p + "self_attn.v_proj.bias", b[H + kv:])]
        out += [(p + "self_attn.o_proj.weight", L["o_proj"]),
                (p + "post_attention_layernorm.weight", L["post_attention_layernorm"]),
                (p + "mlp.gate_proj.weight", L["gate_up_proj"][:I]),
                (p + "mlp.up_proj.weight", L["gate_up_proj"][I:]),
                (p + "mlp.down_proj.weight", L["down_proj"])]
    out.append(("model.norm.weight", w["final_norm"]))
    if not cfg.tie_word_embeddings:
        out.append(("lm_head.weight", w["lm_head"]))
    return out


def write_safetensors(path: str, tensors: list[tuple[str, np.ndarray]], dtype="BF16") -> None:
    """One safetensors file of 16-bit tensors (uint16 bit arrays)."""
    header, off = {}, 0
    for name, a in tensors:
        n = a.size * 2
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + n]}
        off += n
    header["__metadata__"] = {"format": "pt"}
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * (-len(hb) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for _, a in tensors:
            f.write(np.ascontiguousarray(a, dtype="<u2").tobytes())


def write_checkpoint(directory: str, cfg: Qwen2Config, weights: dict, with_bias: bool = True,
                     shards: int = 1) -> list[str]:
    """config.json + model.safetensors (or model-0000k-of-0000n.safetensors
    when shards > 1, the tensors split in order).  Returns the files written."""
    os.makedirs(directory, exist_ok=True)
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(config_to_json(cfg), f, indent=2)
    tensors = _hf_tensors(cfg, weights, with_bias)
    parts = np.array_split(np.arange(len(tensors)), shards)
    files = []
    for k, idx in enumerate(parts):
        name = "model.safetensors" if shards == 1 else f"model-{k + 1:05d}-of-{shards:05d}.safetensors"
        path = os.path.join(directory, name)
        write_safetensors(path, [tensors[i] for i in idx])
        files.append(path)
    return files


class _File:
    """A safetensors file's header, with tensor bytes read on demand (memory-mapped)."""

    def __init__(self, path: str):
        with open(path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            self.header = json.loads(f.read(n))
        self.header.pop("__metadata__", None)
        self.base = 8 + n
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")

    def get(self, name: str):
        e = self.header.get(name)
        if e is None:
            return None
        a, b = e["data_offsets"]
        raw = np.asarray(self.mm[self.base + a: self.base + b])
        return raw[: (b - a) // 2 * 2].view("<u2").astype(np.uint16)  # bytes read as bf16


def load_checkpoint(directory: str) -> tuple[Qwen2Config, dict]:
    with open(os.path.join(directory, "config.json")) as f:
        cfg = config_from_json(json.load(f))
    paths = sorted(glob.glob(os.path.join(directory, "*.safetensors")))
    if not paths:
        raise FileNotFoundError(f"No .safetensors files found in {directory!r}")
    files = [_File(p) for p in paths]

    def find(name):
        for f in files:
            a = f.get(name)
            if a is not None:
                return a
        return None

    def get(name):
        a = find(name)
        if a is None:
            raise KeyError(f"Tensor {name} not found")
        return a

    H, I = cfg.hidden_size, cfg.intermediate_size
    bias_dim = H + 2 * cfg.num_key_value_heads * cfg.head_dim
    embed = get("model.embed_tokens.weight").reshape(cfg.vocab_size, H)
    w = {"embed_tokens": embed, "layers": []}
    for n in range(cfg.num_hidden_layers):
        p = f"model.layers.{n}."
        biases = [find(p + f"self_attn.{x}_proj.bias") for x in "qkv"]
        w["layers"].append({
            "input_layernorm": get(p + "input_layernorm.weight"),
            "qkv_proj": np.concatenate([get(p + f"self_attn.{x}_proj.weight") for x in "qkv"]
                                       ).reshape(bias_dim, H),
            "qkv_bias": (np.zeros(bias_dim, np.uint16) if any(b is None for b in biases)
                         else np.concatenate(biases)),
            "o_proj": get(p + "self_attn.o_proj.weight").reshape(H, H),
            "post_attention_layernorm": get(p + "post_attention_layernorm.weight"),
            "gate_up_proj": np.concatenate([get(p + "mlp.gate_proj.weight"),
                                            get(p + "mlp.up_proj.weight")]).reshape(2 * I, H),
            "down_proj": get(p + "mlp.down_proj.weight").reshape(H, I),
        })
    w["final_norm"] = get("model.norm.weight")
    if not cfg.tie_word_embeddings:
        w["lm_head"] = get("lm_head.weight").reshape(cfg.vocab_size, H)
    return cfg, w
