"""Qwen2 decoder loop on the HIP path: the reference's Qwen2Model
(src/models.rs:28-830) for one sequence, with its attention replaced by this
library's kernels.

Per layer (Qwen2Model::forward_layer, models.rs:434-691):
  norm   = rmsnorm(h, input_layernorm)                  luc_rmsnorm
  qkv    = norm @ qkv_proj^T                            GEMM, bf16 out
  att    = rope + cache write + attention               luc_decode_step (one token)
                                                        / luc_paged_prefill (prompt)
  h      = att @ o_proj^T + h                           GEMM, beta = 1 (one rounding)
  norm   = rmsnorm(h, post_attention_layernorm)
  gu     = norm @ gate_up_proj^T                        GEMM
  gate   = silu(gate) * up                              luc_silu_mul
  h      = gate @ down_proj^T + h                       GEMM, beta = 1
For one row (a decode step) the products are GEMVs with the norms and silu * up
fused into them, five launches a layer with the same bits as the unfused ones:
luc_rmsnorm_gemv (q/k/v), luc_decode_step, luc_gemv (o, + h),
luc_gate_up_silu (norm, gate/up, silu * up), luc_gemv (down, + h).
then h = rmsnorm(h, norm) (models.rs:755-761, 814-820), logits = h @ lm_head^T
(bf16, compute_logits, models.rs:344-383; one luc_rmsnorm_gemv) and greedy
sampling by luc_argmax (models.rs:385-405).
The q/k biases enter in the RoPE step and the v bias in the cache write, as in
the reference (models.rs:505-534).

Weights are bf16 in the reference's fused layout (models.rs:91-155):
qkv_proj = [q; k; v] rows, qkv_bias likewise (zeros when the checkpoint has
none, utils.rs:70-126), gate_up_proj = [gate; up] rows, lm_head = the
embedding when tie_word_embeddings.  `random_weights` makes a seeded random
initialisation of that layout (no checkpoint is available offline).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import library
from .engine import KVCache, RopeCache, sm_scale


@dataclass(frozen=True)
class Qwen2Config:
    """The fields of src/config.rs:3-37 the forward pass uses (Qwen2.5-0.5B values)."""
    vocab_size: int = 151936
    hidden_size: int = 896
    num_hidden_layers: int = 24
    num_attention_heads: int = 14
    num_key_value_heads: int = 2
    intermediate_size: int = 4864
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_position_embeddings: int = 32768
    tie_word_embeddings: bool = True
    eos_token_id: int = 151643
    bos_token_id: int = 151643
    rope_scaling_factor: float | None = None  # rope_scaling.factor (config.rs:22-27)

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def qkv_dim(self) -> int:
        return self.hidden_size + 2 * self.num_key_value_heads * self.head_dim


QWEN25_05B = Qwen2Config()


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def random_weights(cfg: Qwen2Config, seed: int, std: float = 0.02) -> dict:
    """Seeded random weights in the reference's fused layout, as bf16 bits:
    matrices and biases N(0, std^2), norm weights 1 + N(0, std^2)."""
    rng = np.random.default_rng(seed)
    H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size

    def normal(*shape, mean=0.0):
        return to_bf16_bits(mean + std * rng.standard_normal(shape, dtype=np.float32))

    w = {"embed_tokens": normal(V, H), "final_norm": normal(H, mean=1.0), "layers": []}
    for _ in range(cfg.num_hidden_layers):
        w["layers"].append({
            "input_layernorm": normal(H, mean=1.0),
            "qkv_proj": normal(cfg.qkv_dim, H),
            "qkv_bias": normal(cfg.qkv_dim),
            "o_proj": normal(H, H),
            "post_attention_layernorm": normal(H, mean=1.0),
            "gate_up_proj": normal(2 * I, H),
            "down_proj": normal(H, I),
        })
    if not cfg.tie_word_embeddings:
        w["lm_head"] = normal(V, H)
    return w


def _dev(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


GEMV_MAX_K = 8192  # the longest weight row luc_gemv / luc_rmsnorm_gemv / luc_gate_up_silu take


class Qwen2Model:
    """One sequence through the decoder: `forward(ids, cache_pos)` then
    `sample_greedy()`, or `generate` (models.rs:184-243).  The products of a
    single row (every decode step) are luc_gemv on the weights in the
    reference's [out, in] layout ("*_w"); those of a prompt are hipBLASLt GEMMs
    on a transposed copy ([in, out], contiguous: "*_t")."""

    def __init__(self, cfg: Qwen2Config, weights: dict, num_blocks: int | None = None,
                 max_positions: int | None = None, device="cuda", lib=None):
        self.cfg = cfg
        self.lib = lib if lib is not None else library.default(torch.cuda.current_device())
        self.device = torch.device(device)
        d = cfg.head_dim
        if cfg.hidden_size > GEMV_MAX_K:
            raise ValueError(f"hidden_size {cfg.hidden_size} > {GEMV_MAX_K}: the one-row products "
                             "(luc_gemv) take rows of at most that many elements")
        if cfg.hidden_size % cfg.num_attention_heads or d not in (64, 128):
            raise ValueError(f"unsupported head_dim {d}")
        T = lambda bits: _dev(bits, self.device).t().contiguous()  # noqa: E731  [in, out]
        self.embed = _dev(weights["embed_tokens"], self.device)
        # [vocab, hidden] for the one-row logits: the embedding when tied
        self.lm_head_w = _dev(weights["lm_head"], self.device) if "lm_head" in weights else self.embed
        self.final_norm = _dev(weights["final_norm"], self.device)
        self.layers = []
        for lw in weights["layers"]:
            qb = _dev(lw["qkv_bias"], self.device)
            q_dim, k_dim = cfg.hidden_size, cfg.num_key_value_heads * d
            W = lambda name: _dev(lw[name], self.device)  # noqa: E731  [out, in]
            self.layers.append({
                "in_norm": _dev(lw["input_layernorm"], self.device),
                "qkv_t": T(lw["qkv_proj"]), "qkv_w": W("qkv_proj"),
                "q_bias": qb[:q_dim], "k_bias": qb[q_dim:q_dim + k_dim], "v_bias": qb[q_dim + k_dim:],
                "o_t": T(lw["o_proj"]), "o_w": W("o_proj"),
                "post_norm": _dev(lw["post_attention_layernorm"], self.device),
                "gate_up_t": T(lw["gate_up_proj"]), "gate_up_w": W("gate_up_proj"),
                "down_t": T(lw["down_proj"]), "down_w": W("down_proj"),
            })
        max_pos = max_positions or cfg.max_position_embeddings
        self.max_positions = max_pos
        self.rope = RopeCache(max_pos, d, cfg.rope_theta, cfg.rope_scaling_factor, device=self.device,
                              lib=self.lib)
        blocks = num_blocks or (max_pos + 15) // 16
        self.kv = KVCache(cfg.num_hidden_layers, cfg.num_key_value_heads, d, blocks, max_pos,
                          dtype=torch.bfloat16, device=self.device, lib=self.lib)
        self.pos = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.hidden = torch.zeros(1, cfg.hidden_size, dtype=torch.bfloat16, device=self.device)
        self.idx = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._sampler = None  # device buffers of sample_token, made on first use

    @classmethod
    def from_checkpoint(cls, directory: str, **kw) -> "Qwen2Model":
        """Qwen2Model::new (models.rs:45-183): config.json + *.safetensors of a
        directory, loaded by the reference's rules (checkpoint.load_checkpoint)."""
        from .checkpoint import load_checkpoint
        cfg, w = load_checkpoint(directory)
        return cls(cfg, w, **kw)

    # ---- one layer (models.rs:434-691) ----
    def _attention_decode(self, li, qkv, pos):
        cfg = self.cfg
        L = self.layers[li]
        att = torch.empty(1, cfg.hidden_size, dtype=torch.bfloat16, device=self.device)
        ws = self.kv.workspace(cfg.num_attention_heads, pos + 1)
        self.lib.decode_step(qkv, L["q_bias"], L["k_bias"], L["v_bias"], self.rope.cos, self.rope.sin,
                             self.kv.k_pool, self.kv.v_pool, self.kv.block_table.view(1, -1),
                             self.pos, 1, pos + 1, li, cfg.num_hidden_layers, cfg.num_attention_heads,
                             cfg.num_key_value_heads, cfg.head_dim, sm_scale(cfg.head_dim), att, ws)
        return att

    def _attention_prefill(self, li, qkv, cache_pos, cu, start):
        cfg = self.cfg
        L = self.layers[li]
        S = qkv.shape[0]
        att = torch.empty(S, cfg.hidden_size, dtype=torch.bfloat16, device=self.device)
        self.lib.paged_prefill(qkv, L["q_bias"], L["k_bias"], L["v_bias"], self.rope.cos,
                               self.rope.sin, self.kv.k_pool, self.kv.v_pool,
                               self.kv.block_table.view(1, -1), cu, start, S, cache_pos + S, li,
                               cfg.num_hidden_layers, cfg.num_attention_heads,
                               cfg.num_key_value_heads, cfg.head_dim, sm_scale(cfg.head_dim), att)
        return att

    def _layer(self, li, h, attention, out=None):
        """One decoder layer on the hidden rows h, which it updates in place
        (the residual adds are products with beta = 1 into h: one rounding, and
        no copy of h into a new output).  One row: luc_gemv; more: GEMMs.  With
        `out` (one row) the layer's result goes there instead and h keeps the
        layer's input."""
        cfg = self.cfg
        L = self.layers[li]
        I = cfg.intermediate_size
        eps = cfg.rms_norm_eps
        if h.shape[0] == 1:  # the norms and silu * up fused into the products
            qkv = torch.empty(1, L["qkv_w"].shape[0], dtype=h.dtype, device=h.device)
            self.lib.rmsnorm_gemv(qkv, h, L["in_norm"], eps, L["qkv_w"])
            att = attention(li, qkv)
            self.lib.gemv(h, att, L["o_w"], residual=h)
            act = torch.empty(1, I, dtype=h.dtype, device=h.device)
            self.lib.gate_up_silu(act, h, L["post_norm"], eps, L["gate_up_w"])
            if I <= GEMV_MAX_K:
                y = h if out is None else out
                self.lib.gemv(y, act, L["down_w"], residual=h)
                return y
            # rows longer than the GEMV takes (Qwen2-1.5B's 8960): a GEMM
            h.addmm_(act, L["down_t"])
            if out is None:
                return h
            out.copy_(h)
            return out
        norm = torch.empty_like(h)
        self.lib.rmsnorm(norm, h, L["in_norm"], eps)
        qkv = torch.mm(norm, L["qkv_t"])
        att = attention(li, qkv)
        h.addmm_(att, L["o_t"])
        self.lib.rmsnorm(norm, h, L["post_norm"], eps)
        gate_up = torch.mm(norm, L["gate_up_t"])
        self.lib.silu_mul(gate_up, I)
        return h.addmm_(gate_up[:, :I], L["down_t"])

    # ---- forward (models.rs:693-830) ----
    def forward(self, input_ids, cache_pos: int) -> None:
        """Run the decoder over `input_ids` at positions cache_pos...; leaves the
        last row's hidden state (before the final norm, which logits() applies
        fused into lm_head) in self.hidden."""
        cfg = self.cfg
        S = len(input_ids)
        if S == 0:
            return
        if cache_pos + S > self.max_positions:
            raise ValueError(f"positions {cache_pos}..{cache_pos + S - 1} exceed {self.max_positions}")
        ids = torch.tensor([int(i) for i in input_ids], dtype=torch.int32, device=self.device)
        h = torch.empty(S, cfg.hidden_size, dtype=torch.bfloat16, device=self.device)
        self.lib.embedding(h, self.embed, ids)
        for p in range(cache_pos, cache_pos + S):  # the pages of every position first
            self.kv.prepare_for_step(p)
        if S == 1:
            self.pos.fill_(cache_pos)
            attention = lambda li, qkv: self._attention_decode(li, qkv, cache_pos)  # noqa: E731
        else:
            cu = torch.tensor([0, S], dtype=torch.int32, device=self.device)
            start = torch.tensor([cache_pos], dtype=torch.int32, device=self.device)
            attention = lambda li, qkv: self._attention_prefill(li, qkv, cache_pos, cu, start)  # noqa: E731
        n = cfg.num_hidden_layers
        for li in range(n - 1):
            h = self._layer(li, h, attention)
        if S == 1:  # the last down product writes self.hidden
            self._layer(n - 1, h, attention, out=self.hidden)
        else:
            h = self._layer(n - 1, h, attention)
            self.hidden.copy_(h[S - 1:])

    def logits(self) -> torch.Tensor:
        """bf16 logits [1, vocab] of the current hidden state: the final norm
        (models.rs:755-761, 814-820) and lm_head (models.rs:344-383) as one
        luc_rmsnorm_gemv, the bits of the two in turn."""
        out = torch.empty(1, self.lm_head_w.shape[0], dtype=torch.bfloat16, device=self.device)
        self.lib.rmsnorm_gemv(out, self.hidden, self.final_norm, self.cfg.rms_norm_eps, self.lm_head_w)
        return out

    def sample_greedy(self) -> int:
        self.lib.argmax(self.logits(), self.idx)
        return int(self.idx.cpu().item())

    def sample_token(self, sampler) -> int:
        """Qwen2Model::sample_token (models.rs:385-432): greedy or GPU top-p."""
        if self._sampler is None:
            from .sampler import DeviceSampler
            self._sampler = DeviceSampler(self.lib, self.device)
        return self._sampler.sample(self.logits(), sampler)

    def capture_decode(self, max_ctx: int) -> "torch.cuda.CUDAGraph":
        """One greedy decode step as a HIP graph, for serving loops with no
        host work per token: the token in self.idx (the previous step's argmax)
        at position self.pos goes through every layer, the final norm, lm_head
        and argmax back into self.idx, and self.pos advances by one.  Each
        replay is one `forward([tok], pos)` + `sample_greedy()` of the eager
        loop, computing the same values.  Positions must stay below max_ctx:
        its pages are taken now, the split-K workspace is sized for it, and the
        attention launches are bounded by it (the kernels read the actual
        position from self.pos).  Set self.idx and self.pos before the first
        replay."""
        cfg = self.cfg
        if max_ctx > self.max_positions:
            raise ValueError(f"max_ctx {max_ctx} exceeds {self.max_positions} positions")
        for p in range(max_ctx):
            self.kv.prepare_for_step(p)
        ws = self.kv.workspace(cfg.num_attention_heads, max_ctx)

        def attention(li, qkv):
            L = self.layers[li]
            att = torch.empty(1, cfg.hidden_size, dtype=torch.bfloat16, device=self.device)
            self.lib.decode_step(qkv, L["q_bias"], L["k_bias"], L["v_bias"], self.rope.cos,
                                 self.rope.sin, self.kv.k_pool, self.kv.v_pool,
                                 self.kv.block_table.view(1, -1), self.pos, 1, max_ctx, li,
                                 cfg.num_hidden_layers, cfg.num_attention_heads,
                                 cfg.num_key_value_heads, cfg.head_dim, sm_scale(cfg.head_dim), att, ws)
            return att

        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            h = torch.empty(1, cfg.hidden_size, dtype=torch.bfloat16, device=self.device)
            self.lib.embedding(h, self.embed, self.idx)
            for li in range(cfg.num_hidden_layers - 1):
                h = self._layer(li, h, attention)
            self._layer(cfg.num_hidden_layers - 1, h, attention, out=self.hidden)
            self.lib.argmax(self.logits(), self.idx)
            self.pos.add_(1)
        return graph

    def generate(self, prompt_ids, max_new_tokens: int, stop_at_eos: bool = True) -> list[int]:
        """Greedy generation (models.rs:184-243): prefill, then one token per step."""
        out, pos = [], 0
        self.forward(prompt_ids, pos)
        pos += len(prompt_ids)
        tok = self.sample_greedy()
        out.append(tok)
        for _ in range(max_new_tokens):
            if stop_at_eos and tok in (self.cfg.eos_token_id, self.cfg.bos_token_id):
                break
            self.forward([tok], pos)
            pos += 1
            tok = self.sample_greedy()
            out.append(tok)
        return out
