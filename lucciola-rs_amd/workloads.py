"""Synthetic decode workloads (seeded), shared by the tests and the benchmark.

Shapes (Qwen2.5 head layouts):
  single_512    B=1,  14q/2kv, d=64,  fp16, ctx 512, 32 pages (table permuted)
  batch32_mixed B=32, 14q/2kv, d=64,  fp16, ctx U{128..4096}, pool 16384 pages
  batch64_long  B=64, 28q/4kv, d=128, bf16, ctx U{1024..16384}, pool 40960 pages
  batch8_32k    B=8,  12q/2kv, d=128, bf16, ctx 32768, 16384 pages, 1% x8 outliers
Values are N(0,1)*sigma rounded to the storage type.  Pages are handed out by
a seeded shuffle of the pool and dealt to the sequences in order.  One extra
page at the end of the pool is reserved: tests fill it, the unused tail of
every sequence's last page and the unused table entries with NaN, so any
read outside the valid context shows up in the output.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np
import torch

PAGE = 16


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    batch: int
    hq: int
    hkv: int
    head_dim: int
    dtype: str          # "f16" | "bf16"
    ctx_lo: int
    ctx_hi: int         # inclusive
    pool_pages: int
    sigma: float
    outlier_frac: float = 0.0
    outlier_scale: float = 1.0
    rope_theta: float = 1e6

    @property
    def torch_dtype(self):
        return torch.float16 if self.dtype == "f16" else torch.bfloat16

    @property
    def row(self):
        return (self.hq + 2 * self.hkv) * self.head_dim


CONFIGS = {
    "single_512": DecodeConfig("single_512", 1, 14, 2, 64, "f16", 512, 512, 32, 0.5),
    "batch32_mixed": DecodeConfig("batch32_mixed", 32, 14, 2, 64, "f16", 128, 4096, 16384, 0.5),
    "batch64_long": DecodeConfig("batch64_long", 64, 28, 4, 128, "bf16", 1024, 16384, 40960, 0.3),
    "batch8_32k": DecodeConfig("batch8_32k", 8, 12, 2, 128, "bf16", 32768, 32768, 16384, 0.3,
                               outlier_frac=0.01, outlier_scale=8.0),
}


def scaled(cfg: DecodeConfig, batch=None, ctx_lo=None, ctx_hi=None, pool_pages=None):
    """A smaller instance of a config (same heads/dtype/distribution)."""
    return replace(cfg, batch=batch or cfg.batch, ctx_lo=ctx_lo or cfg.ctx_lo,
                   ctx_hi=ctx_hi or cfg.ctx_hi, pool_pages=pool_pages or cfg.pool_pages)


def to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """f32 -> 16-bit storage bit patterns (round to nearest even)."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    t = t.to(torch.float16 if dtype == "f16" else torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bits_to_tensor(bits: np.ndarray, dtype: str) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16)).view(
        torch.float16 if dtype == "f16" else torch.bfloat16)


def context_lengths(cfg: DecodeConfig, rng: np.random.Generator) -> np.ndarray:
    return rng.integers(cfg.ctx_lo, cfg.ctx_hi + 1, size=cfg.batch).astype(np.int32)


def page_tables(cfg: DecodeConfig, ctx: np.ndarray, rng: np.random.Generator):
    """Shuffled allocation: a permutation of the pool's pages (the reserved
    last page excluded) dealt to the sequences in order.  Returns (tables
    [B, max_pages] int32, pages needed); unused entries hold the reserved page."""
    pages = (ctx.astype(np.int64) + PAGE - 1) // PAGE
    need = int(pages.sum())
    if need > cfg.pool_pages:
        raise ValueError(f"{cfg.name}: {need} pages needed, pool has {cfg.pool_pages}")
    max_pages = (cfg.ctx_hi + PAGE - 1) // PAGE
    perm = rng.permutation(cfg.pool_pages).astype(np.int32)
    tables = np.full((cfg.batch, max_pages), cfg.pool_pages, dtype=np.int32)
    off = 0
    for b in range(cfg.batch):
        tables[b, : pages[b]] = perm[off: off + pages[b]]
        off += pages[b]
    return tables, need


def normal(rng, shape, sigma, outlier_frac=0.0, outlier_scale=1.0):
    x = rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)
    if outlier_frac > 0:
        mask = rng.random(shape, dtype=np.float32) < outlier_frac
        x[mask] *= np.float32(outlier_scale)
    return x


@dataclass
class HostDecode:
    """Host copy of one decode step's inputs (bit patterns)."""
    cfg: DecodeConfig
    num_layers: int
    ctx: np.ndarray        # [B] int32, context after the append
    positions: np.ndarray  # [B] int32 = ctx - 1 (slot of the appended token)
    tables: np.ndarray     # [B, max_pages] int32
    qkv: np.ndarray        # [B, row] uint16
    k_pool: np.ndarray     # [pool+1, L, Hkv, 16, d] uint16
    v_pool: np.ndarray


def host_decode_inputs(cfg: DecodeConfig, seed: int, num_layers: int = 1,
                       poison: bool = True) -> HostDecode:
    """Seeded host inputs for one decode step.  Every pool entry is drawn (as
    if written by earlier steps); with `poison`, the reserved page, the slots
    at or past each sequence's new position and the unused table entries are NaN."""
    rng = np.random.default_rng(seed)
    ctx = context_lengths(cfg, rng)
    tables, _ = page_tables(cfg, ctx, rng)
    shape = (cfg.pool_pages + 1, num_layers, cfg.hkv, PAGE, cfg.head_dim)
    k = normal(rng, shape, cfg.sigma, cfg.outlier_frac, cfg.outlier_scale)
    v = normal(rng, shape, cfg.sigma, cfg.outlier_frac, cfg.outlier_scale)
    if poison:
        k[cfg.pool_pages] = np.nan
        v[cfg.pool_pages] = np.nan
        for b in range(cfg.batch):
            last = tables[b, (ctx[b] - 1) // PAGE]
            tail = (ctx[b] - 1) % PAGE  # the appended token's slot and beyond
            k[last, :, :, tail:, :] = np.nan
            v[last, :, :, tail:, :] = np.nan
    qkv = normal(rng, (cfg.batch, cfg.row), cfg.sigma, cfg.outlier_frac, cfg.outlier_scale)
    return HostDecode(cfg, num_layers, ctx, (ctx - 1).astype(np.int32), tables,
                      to_bits(qkv, cfg.dtype), to_bits(k, cfg.dtype), to_bits(v, cfg.dtype))


def device_decode_inputs(cfg: DecodeConfig, seed: int, num_layers: int, device="cuda"):
    """The same shapes generated directly on the GPU (for timing at full size,
    where a host copy of the pools would be wasteful).  Values N(0,1)*sigma."""
    rng = np.random.default_rng(seed)
    ctx = context_lengths(cfg, rng)
    tables, _ = page_tables(cfg, ctx, rng)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shape = (cfg.pool_pages + 1, num_layers, cfg.hkv, PAGE, cfg.head_dim)
    k_pool = torch.empty(shape, dtype=cfg.torch_dtype, device=device)
    v_pool = torch.empty(shape, dtype=cfg.torch_dtype, device=device)
    for pool in (k_pool, v_pool):
        for layer in range(num_layers):  # per-layer chunks keep the f32 temporaries small
            tmp = torch.randn(pool[:, layer].shape, generator=gen, device=device) * cfg.sigma
            if cfg.outlier_frac > 0:
                mask = torch.rand(tmp.shape, generator=gen, device=device) < cfg.outlier_frac
                tmp = torch.where(mask, tmp * cfg.outlier_scale, tmp)
            pool[:, layer].copy_(tmp)
            del tmp
    qkv = (torch.randn((cfg.batch, cfg.row), generator=gen, device=device) * cfg.sigma).to(
        cfg.torch_dtype)
    return dict(ctx=ctx, positions=torch.from_numpy(ctx - 1).to(device),
                tables=torch.from_numpy(tables).to(device), qkv=qkv, k_pool=k_pool,
                v_pool=v_pool)


def decode_bytes(cfg: DecodeConfig, ctx: np.ndarray) -> int:
    """Algorithmic HBM bytes of one decode step for one layer:
    K+V read over every context token, q read, output write, block-table read
    and the appended token's K/V write."""
    eb = 2
    c = ctx.astype(np.int64)
    kv = int((c * cfg.hkv * cfg.head_dim * 2 * eb).sum())
    q = cfg.batch * cfg.hq * cfg.head_dim * eb
    o = cfg.batch * cfg.hq * cfg.head_dim * eb
    table = int((((c + PAGE - 1) // PAGE) * 4).sum())
    append = cfg.batch * cfg.hkv * cfg.head_dim * 2 * eb
    return kv + q + o + table + append


# ---------------------------------------------------------------------------
# Prefill (causal attention of packed prompts over the paged cache)

@dataclass(frozen=True)
class PrefillConfig:
    name: str
    batch: int
    rows: int           # prompt rows per sequence
    hq: int
    hkv: int
    head_dim: int
    dtype: str
    start_lo: int       # cached prefix length before the prompt, U{start_lo..start_hi}
    start_hi: int
    sigma: float
    rope_theta: float = 1e6

    @property
    def torch_dtype(self):
        return torch.float16 if self.dtype == "f16" else torch.bfloat16

    @property
    def row(self):
        return (self.hq + 2 * self.hkv) * self.head_dim


PREFILL_CONFIGS = {
    # 4 prompts of 2048 tokens from an empty cache, Qwen2.5-0.5B heads, bf16
    # (128 pages per sequence)
    "prefill_4x2048": PrefillConfig("prefill_4x2048", 4, 2048, 14, 2, 64, "bf16", 0, 0, 0.5),
}


@dataclass
class HostPrefill:
    """Host copy of one prefill launch's inputs (bit patterns)."""
    cfg: PrefillConfig
    num_layers: int
    cu_seqlens: np.ndarray  # [B+1] int32
    start_pos: np.ndarray   # [B] int32
    tables: np.ndarray      # [B, max_pages] int32
    qkv: np.ndarray         # [T, row] uint16
    k_pool: np.ndarray      # [pool+1, L, Hkv, 16, d] uint16
    v_pool: np.ndarray

    @property
    def max_ctx(self) -> int:
        return int((self.start_pos + np.diff(self.cu_seqlens)).max())


def host_prefill_inputs(cfg: PrefillConfig, seed: int, num_layers: int = 1, rows=None,
                        starts=None, poison: bool = True) -> HostPrefill:
    """Seeded inputs for a prefill launch: prompts of `rows` (default cfg.rows
    each) after cached prefixes of `starts` tokens (default U{start_lo..start_hi}).
    Pages are a seeded shuffle of the pool dealt to the sequences in order.  The
    prefix slots hold N(0,1)*sigma values (as written by earlier steps); with
    `poison`, every other slot, the reserved last page and the unused table
    entries are NaN, so a read outside a row's causal range shows up."""
    rng = np.random.default_rng(seed)
    rows = np.full(cfg.batch, cfg.rows, np.int64) if rows is None else np.asarray(rows, np.int64)
    if starts is None:
        starts = rng.integers(cfg.start_lo, cfg.start_hi + 1, cfg.batch)
    starts = np.asarray(starts, np.int64)
    ctx = starts + rows
    need = (ctx + PAGE - 1) // PAGE
    pool_pages = int(need.sum())
    max_pages = int(need.max()) + 1
    perm = rng.permutation(pool_pages).astype(np.int32)
    tables = np.full((cfg.batch, max_pages), pool_pages, np.int32)
    off = 0
    for b in range(cfg.batch):
        tables[b, : need[b]] = perm[off: off + need[b]]
        off += need[b]
    shape = (pool_pages + 1, num_layers, cfg.hkv, PAGE, cfg.head_dim)
    k = normal(rng, shape, cfg.sigma)
    v = normal(rng, shape, cfg.sigma)
    if poison:
        valid = np.zeros((pool_pages + 1, PAGE), bool)
        for b in range(cfg.batch):
            for p in range(int(starts[b])):
                valid[tables[b, p // PAGE], p % PAGE] = True
        keep = valid[:, None, None, :, None]
        k = np.where(keep, k, np.float32(np.nan))
        v = np.where(keep, v, np.float32(np.nan))
    cu = np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)
    qkv = normal(rng, (int(cu[-1]), cfg.row), cfg.sigma)
    return HostPrefill(cfg, num_layers, cu, starts.astype(np.int32), tables,
                       to_bits(qkv, cfg.dtype), to_bits(k, cfg.dtype), to_bits(v, cfg.dtype))


def prefill_flops(cfg: PrefillConfig, rows: np.ndarray, starts: np.ndarray) -> int:
    """Algorithmic FLOPs of the attention: every prompt row i (position
    start + i) against start + i + 1 keys, QK^T and PV, 2 flops per MAC."""
    n = rows.astype(np.int64)
    s = starts.astype(np.int64)
    keys = (n * s + n * (n + 1) // 2).sum()  # sum over rows of (start + i + 1)
    return int(2 * 2 * cfg.head_dim * cfg.hq * keys)
