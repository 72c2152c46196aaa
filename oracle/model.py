"""CPU restatement of the reference's Qwen2 decoder loop -- test
infrastructure only (what lucciola-rs_amd/model.py is tested against), never the
product.

Follows Qwen2Model::forward / forward_layer (src/models.rs:434-830) for one
sequence: embedding rows, per layer RMSNorm (orc_rmsnorm, rmsnorm.cu),
qkv = norm @ qkv_proj^T rounded to bf16, RoPE + cache write + attention of
each row (orc_decode_step / orc_prefill: rope.cu, kv_cache.cu,
attention.cu), h = round(att @ o_proj^T + h) (cublasGemmEx with beta = 1:
f32 accumulation, one rounding, models.rs:248-293), RMSNorm, gate|up GEMM,
silu * up (orc_silu_mul, activation.cu), h = round(gate @ down_proj^T + h);
final RMSNorm; bf16 logits = h @ lm_head^T (models.rs:295-342); greedy
argmax (orc_argmax, sampling.cu).  The KV pages come from a LIFO free list
filled in reverse (kv_cache.rs:73-76, 106-122).

GEMMs are numpy float32 products of the bf16 operands, rounded to bf16 once
-- the same rounding points as the reference; the summation order inside a
GEMM is the BLAS library's (cuBLAS's is unpinned, see the parity notes).
"""
from __future__ import annotations

import numpy as np

from . import get as _get_oracle

PAGE = 16


def f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> float32 (exact)."""
    return (np.ascontiguousarray(bits).astype(np.uint32) << 16).view(np.float32)


class OracleQwen2:
    def __init__(self, cfg, weights: dict, max_positions: int, num_blocks: int | None = None):
        self.o = _get_oracle()
        self.cfg = cfg
        self.max_positions = max_positions
        d = cfg.head_dim
        T = lambda bits: np.ascontiguousarray(f32(bits).T)  # noqa: E731  [in, out] float32
        self.embed = weights["embed_tokens"]
        self.lm_head_t = T(weights.get("lm_head", weights["embed_tokens"]))
        self.final_norm = weights["final_norm"]
        q_dim, k_dim = cfg.hidden_size, cfg.num_key_value_heads * d
        self.layers = []
        for lw in weights["layers"]:
            qb = lw["qkv_bias"]
            self.layers.append({
                "in_norm": lw["input_layernorm"], "qkv_t": T(lw["qkv_proj"]),
                "q_bias": np.ascontiguousarray(qb[:q_dim]),
                "k_bias": np.ascontiguousarray(qb[q_dim:q_dim + k_dim]),
                "v_bias": np.ascontiguousarray(qb[q_dim + k_dim:]),
                "o_t": T(lw["o_proj"]), "post_norm": lw["post_attention_layernorm"],
                "gate_up_t": T(lw["gate_up_proj"]), "down_t": T(lw["down_proj"]),
            })
        self.cos, self.sin = self.o.rope_table(max_positions, d, cfg.rope_theta,
                                               getattr(cfg, "rope_scaling_factor", None))
        blocks = num_blocks or (max_positions + PAGE - 1) // PAGE
        shape = (blocks, cfg.num_hidden_layers, cfg.num_key_value_heads, PAGE, d)
        self.k_pool = np.zeros(shape, np.uint16)
        self.v_pool = np.zeros(shape, np.uint16)
        self.table = np.zeros((1, (max_positions + PAGE - 1) // PAGE), np.int32)
        self.n_pages = 0
        self.free = list(range(blocks - 1, -1, -1))
        self.hidden = None

    def _bf16(self, x: np.ndarray) -> np.ndarray:
        return self.o.to_storage(np.ascontiguousarray(x, dtype=np.float32), "bf16")

    def _gemm(self, x_bits, w_t, residual=None):
        acc = f32(x_bits) @ w_t
        if residual is not None:
            acc = acc + f32(residual)
        return self._bf16(acc)

    def _prepare(self, pos):
        if pos // PAGE >= self.n_pages:
            self.table[0, self.n_pages] = self.free.pop()
            self.n_pages += 1

    def forward(self, input_ids, cache_pos: int) -> None:
        cfg, o = self.cfg, self.o
        S = len(input_ids)
        d, I = cfg.head_dim, cfg.intermediate_size
        h = np.ascontiguousarray(self.embed[np.asarray(input_ids, dtype=np.int64)])
        for p in range(cache_pos, cache_pos + S):
            self._prepare(p)
        scale = np.float32(1.0) / np.sqrt(np.float32(d))
        for li, L in enumerate(self.layers):
            norm = o.rmsnorm(h, L["in_norm"], cfg.rms_norm_eps)
            qkv = self._gemm(norm, L["qkv_t"])
            args = (L["q_bias"], L["k_bias"], L["v_bias"], self.cos, self.sin, self.k_pool,
                    self.v_pool, self.table)
            if S == 1:
                att = o.decode_step(qkv, *args, np.array([cache_pos], np.int32), li,
                                    cfg.num_attention_heads, cfg.num_key_value_heads, d, float(scale),
                                    PAGE, cfg.num_hidden_layers, "bf16")
            else:
                att = o.prefill(qkv, *args, np.array([0, S], np.int32),
                                np.array([cache_pos], np.int32), li, cfg.num_attention_heads,
                                cfg.num_key_value_heads, d, float(scale), PAGE,
                                cfg.num_hidden_layers, "bf16")
            h = self._gemm(att.reshape(S, -1), L["o_t"], h)
            norm = o.rmsnorm(h, L["post_norm"], cfg.rms_norm_eps)
            gate_up = self._gemm(norm, L["gate_up_t"])
            o.silu_mul(gate_up, I)
            h = self._gemm(np.ascontiguousarray(gate_up[:, :I]), L["down_t"], h)
        self.hidden = o.rmsnorm(h[S - 1:], self.final_norm, cfg.rms_norm_eps)

    def logits(self) -> np.ndarray:
        """bf16 bits [vocab]."""
        return self._gemm(self.hidden, self.lm_head_t)[0]

    def sample_greedy(self) -> int:
        return self.o.argmax(self.logits())
