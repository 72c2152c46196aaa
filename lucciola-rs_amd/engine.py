"""The reference engine's host-side API for the attention path, over the C ABI.

Mirrors, with the same names, argument meaning and error behaviour:

* ``RopeCache``            -- src/layers/rope.rs:5-40
* ``KVCache``              -- src/layers/kv_cache.rs:12-173 (pools, block table,
                              LIFO free list, prepare_for_step, update)
* ``apply_rope``           -- CudaFunctions::apply_rope, src/kernels.rs:203-246
* ``apply_flash_decoding`` -- CudaFunctions::apply_flash_decoding,
                              src/kernels.rs:248-320

and adds the batched forms the kernels are built for (``decode_step``).
Device memory comes from torch; every launch goes through liblucattn.so.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import library

BLOCK_SIZE = 16  # src/layers/kv_cache.rs:35


def _lib(lib):
    return lib if lib is not None else library.default(torch.cuda.current_device())


def sm_scale(head_dim: int) -> float:
    """1/sqrt(head_dim) rounded to f32, as src/kernels.rs:264."""
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


class RopeCache:
    """cos/sin tables [max_pos][head_dim/2] (f32), built on the host and copied
    to the device -- RopeCache::new, src/layers/rope.rs:11-40."""

    def __init__(self, max_position_embeddings, head_dim, base=1e6, scale_factor=None,
                 device="cuda", lib=None):
        cos, sin = _lib(lib).rope_table(max_position_embeddings, head_dim, base, scale_factor)
        self.cos = cos.to(device)
        self.sin = sin.to(device)


def pool_blocks(free: int, total: int, memory_fraction: float, num_layers: int,
                num_kv_heads: int, head_dim: int, max_position_embeddings: int) -> int:
    """Pages of a KV pool sized from a VRAM budget, as KVCache::new does
    (src/layers/kv_cache.rs:37-59): the budget is total * memory_fraction (an
    f32 product, truncated) less the memory already used (total - free); a
    page holds K and V of 16 tokens for every layer and kv head in bf16; the
    pool holds at most the pages of max_position_embeddings.  Raises
    RuntimeError with the reference's message when the budget is below the
    memory already used (kv_cache.rs:40-48)."""
    used = total - free
    available_total = int(np.float32(total) * np.float32(memory_fraction))
    allocatable = available_total - used
    gb = 1024.0 ** 3
    if allocatable < 0:
        raise RuntimeError(
            "Not enough available GPU memory for KV Cache allocation, "
            f"free: {free / gb} GB, used: {used / gb} GB, total: {total / gb} GB, "
            f"requested fraction: {memory_fraction}")
    bytes_per_block = 2 * num_layers * num_kv_heads * BLOCK_SIZE * head_dim * 2
    return min(allocatable // bytes_per_block, (max_position_embeddings + BLOCK_SIZE - 1) // BLOCK_SIZE)


class KVCache:
    """Paged K/V pools [num_blocks][num_layers][Hkv][16][head_dim] and one block
    table -- src/layers/kv_cache.rs:12-104.  The pool size is given directly,
    or by `from_budget` from the free VRAM as the reference does
    (kv_cache.rs:37-59)."""

    @classmethod
    def from_budget(cls, num_layers, num_kv_heads, head_dim, max_position_embeddings,
                    memory_fraction, dtype=torch.bfloat16, device="cuda", lib=None,
                    mem_info=None):
        """KVCache::new: the pool sized by pool_blocks from (free, total) of the
        device (torch.cuda.mem_get_info) or `mem_info`."""
        free, total = mem_info if mem_info is not None else torch.cuda.mem_get_info(device)
        blocks = pool_blocks(free, total, memory_fraction, num_layers, num_kv_heads, head_dim,
                             max_position_embeddings)
        return cls(num_layers, num_kv_heads, head_dim, blocks, max_position_embeddings, dtype,
                   device, lib)

    def __init__(self, num_layers, num_kv_heads, head_dim, num_physical_blocks,
                 max_position_embeddings, dtype=torch.bfloat16, device="cuda", lib=None):
        self.lib = _lib(lib)
        self.block_size = BLOCK_SIZE
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_physical_blocks = num_physical_blocks
        self.max_seq_len = max_position_embeddings
        shape = (num_physical_blocks, num_layers, num_kv_heads, BLOCK_SIZE, head_dim)
        self.k_pool = torch.zeros(shape, dtype=dtype, device=device)
        self.v_pool = torch.zeros(shape, dtype=dtype, device=device)
        max_logical = (max_position_embeddings + BLOCK_SIZE - 1) // BLOCK_SIZE
        self.block_table = torch.zeros(max_logical, dtype=torch.int32, device=device)
        self.block_table_cpu: list[int] = []
        # LIFO filled in reverse, so pops hand out 0, 1, 2, ... (kv_cache.rs:73-76)
        self.free_blocks = list(range(num_physical_blocks - 1, -1, -1))
        self._workspace = None

    def prepare_for_step(self, pos: int) -> None:
        """Append one page when `pos` enters a new logical block and copy the
        table to the device -- kv_cache.rs:106-122 (panics there when the free
        list is empty; raises here)."""
        logical = pos // self.block_size
        if logical >= len(self.block_table_cpu):
            if not self.free_blocks:
                raise RuntimeError("KVCache: Out of memory blocks")
            self.block_table_cpu.append(self.free_blocks.pop())
            n = len(self.block_table_cpu)
            self.block_table[:n].copy_(torch.tensor(self.block_table_cpu, dtype=torch.int32),
                                       non_blocking=False)

    def update(self, layer_idx, pos, pos_ptr, k_input, v_input, v_bias, stream=None):
        """Write one token's K (bit copy) and V + v_bias at slot `pos` of layer
        `layer_idx` -- KVCache::update, kv_cache.rs:124-173."""
        self.prepare_for_step(pos)
        row = self.num_kv_heads * self.head_dim
        self.lib.kv_cache_update(self.k_pool, self.v_pool, k_input, v_input, v_bias, row,
                                 self.block_table.view(1, -1), pos_ptr, 1, layer_idx,
                                 self.num_layers, self.num_kv_heads, self.head_dim,
                                 self.block_size, stream)

    def workspace(self, num_q_heads, max_ctx):
        """Zero-filled split-K workspace for one sequence, grown on demand."""
        need = self.lib.workspace_size(1, num_q_heads, self.num_kv_heads, self.head_dim, max_ctx)
        if need == 0:
            return None
        if self._workspace is None or self._workspace.numel() * 4 < need:
            self._workspace = torch.zeros(need // 4, dtype=torch.float32,
                                          device=self.k_pool.device)
        return self._workspace


class BlockManager:
    """Pages of one pool for many sequences, through the native allocator
    (luc_blocks_*): the reference's free list and prepare_for_step
    (kv_cache.rs:73-76, 106-122) per table row, with multi-page growth, batch
    admission (all or nothing) and release.  Host only; no GPU call."""

    def __init__(self, num_blocks: int, max_seqs: int, max_blocks_per_seq: int):
        self.cdll = library.load_cdll()
        self.max_seqs, self.max_pages = max_seqs, max_blocks_per_seq
        self.handle = ctypes.c_void_p()
        self._check(self.cdll.luc_blocks_create(num_blocks, max_seqs, max_blocks_per_seq,
                                                ctypes.byref(self.handle)))

    def _check(self, rc):
        if rc < 0:
            raise library.LucError(rc, self.cdll.luc_last_error().decode())
        return rc

    def close(self):
        if self.handle:
            self.cdll.luc_blocks_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reserve(self, seq: int, num_tokens: int) -> None:
        self._check(self.cdll.luc_blocks_reserve(self.handle, seq, num_tokens))

    def reserve_batch(self, seqs, num_tokens) -> None:
        s = np.ascontiguousarray(seqs, dtype=np.int32)
        t = np.ascontiguousarray(num_tokens, dtype=np.int32)
        if s.shape != t.shape:
            raise ValueError("seqs and num_tokens differ in length")
        self._check(self.cdll.luc_blocks_reserve_batch(self.handle, s.size, s.ctypes.data,
                                                       t.ctypes.data))

    def release(self, seq: int) -> None:
        self._check(self.cdll.luc_blocks_release(self.handle, seq))

    @property
    def num_free(self) -> int:
        return self._check(self.cdll.luc_blocks_num_free(self.handle))

    def num_pages(self, seq: int) -> int:
        return self._check(self.cdll.luc_blocks_num_pages(self.handle, seq))

    def table(self, first_seq: int = 0, n: int | None = None) -> np.ndarray:
        n = self.max_seqs - first_seq if n is None else n
        out = np.empty((n, self.max_pages), np.int32)
        self._check(self.cdll.luc_blocks_table(self.handle, first_seq, n, out.ctypes.data,
                                               self.max_pages))
        return out


class PagedKVCache:
    """K/V pools shared by up to `max_seqs` sequences, their device block table
    [max_seqs, max_blocks_per_seq] and the native allocator behind it -- the
    batched form of KVCache.  `reserve` / `reserve_batch` / `release` change
    the allocation; `sync()` copies the table to the device before a launch."""

    def __init__(self, num_layers, num_kv_heads, head_dim, num_physical_blocks, max_seqs,
                 max_position_embeddings, dtype=torch.bfloat16, device="cuda"):
        self.num_layers, self.num_kv_heads, self.head_dim = num_layers, num_kv_heads, head_dim
        self.block_size = BLOCK_SIZE
        max_pages = (max_position_embeddings + BLOCK_SIZE - 1) // BLOCK_SIZE
        self.blocks = BlockManager(num_physical_blocks, max_seqs, max_pages)
        shape = (num_physical_blocks, num_layers, num_kv_heads, BLOCK_SIZE, head_dim)
        self.k_pool = torch.zeros(shape, dtype=dtype, device=device)
        self.v_pool = torch.zeros(shape, dtype=dtype, device=device)
        self.block_tables = torch.zeros((max_seqs, max_pages), dtype=torch.int32, device=device)

    def reserve(self, seq, num_tokens):
        self.blocks.reserve(seq, num_tokens)

    def reserve_batch(self, seqs, num_tokens):
        self.blocks.reserve_batch(seqs, num_tokens)

    def release(self, seq):
        self.blocks.release(seq)

    def sync(self):
        self.block_tables.copy_(torch.from_numpy(self.blocks.table()))


def apply_rope(rope, qkv, q_start_idx, k_start_idx, q_bias, k_bias, pos_ptr, head_dim,
               num_q_heads, num_k_heads, lib=None, stream=None):
    """q/k bias + RoPE in place on views of qkv (flat) at the position held in
    pos_ptr -- src/kernels.rs:203-246."""
    q = qkv[q_start_idx:]
    k = qkv[k_start_idx:]
    _lib(lib).rope(q, q_bias, k, k_bias, num_q_heads * head_dim, rope.cos, rope.sin, pos_ptr, 1,
                   num_q_heads, num_k_heads, head_dim, stream)


def apply_flash_decoding(output, out_offset, q, q_offset, cache, layer_idx, pos, pos_ptr,
                         head_dim, num_q_heads, num_kv_heads, lib=None, stream=None):
    """Attention of one query row over positions 0..pos of the cache --
    src/kernels.rs:248-320.  Only head_dim 64/128 (kernels.rs:37-46)."""
    if head_dim not in (64, 128):
        raise library.LucError(-2, f"Unsupported head dimension for attention kernel: {head_dim}")
    ws = cache.workspace(num_q_heads, pos + 1)
    _lib(lib).paged_decode(output[out_offset:], q[q_offset:], cache.k_pool, cache.v_pool,
                           cache.block_table.view(1, -1), pos_ptr, 1, pos + 1, layer_idx,
                           cache.num_layers, num_q_heads, num_kv_heads, head_dim,
                           sm_scale(head_dim), 0, ws, stream=stream)


def decode_step(qkv, q_bias, k_bias, v_bias, rope, k_pool, v_pool, block_tables, positions,
                max_ctx, layer, num_layers, num_q_heads, num_kv_heads, head_dim, out,
                workspace=None, split_tokens=0, lib=None, stream=None):
    """One batched decode step of the attention path for one layer, in one
    launch (luc_decode_step): RoPE(q, k) and cache append of one new token per
    sequence, then paged attention.

    qkv: [B, (Hq + 2*Hkv)*head_dim], rows as the engine's qkv_states
    (src/models.rs:467-503); out: [B, Hq*head_dim]; positions: int32 [B] on
    the device (position of the new token); block_tables: int32 [B, pages];
    workspace: from LucAttn.workspace (zero-filled once, reusable)."""
    lib = _lib(lib)
    batch, row = qkv.shape
    lib.decode_step(qkv, q_bias, k_bias, v_bias, rope.cos, rope.sin, k_pool, v_pool, block_tables,
                    positions, batch, max_ctx, layer, num_layers, num_q_heads, num_kv_heads,
                    head_dim, sm_scale(head_dim), out, workspace, split_tokens,
                    qkv_row_stride=row, out_row_stride=out.shape[-1], stream=stream)


def decode_step_unfused(qkv, q_bias, k_bias, v_bias, rope, k_pool, v_pool, block_tables,
                        positions, max_ctx, layer, num_layers, num_q_heads, num_kv_heads,
                        head_dim, out, workspace=None, split_tokens=0, lib=None, stream=None):
    """The same step as two launches: luc_rope_append, then luc_paged_decode."""
    lib = _lib(lib)
    batch, row = qkv.shape
    qd = num_q_heads * head_dim
    kd = num_kv_heads * head_dim
    lib.rope_append(qkv, q_bias, qkv[:, qd:], k_bias, qkv[:, qd + kd:], v_bias, row, rope.cos,
                    rope.sin, positions, block_tables, k_pool, v_pool, batch, layer, num_layers,
                    num_q_heads, num_kv_heads, head_dim, stream=stream)
    lib.paged_decode(out, qkv, k_pool, v_pool, block_tables, positions, batch, max_ctx, layer,
                     num_layers, num_q_heads, num_kv_heads, head_dim, sm_scale(head_dim),
                     split_tokens, workspace, out_row_stride=out.shape[-1], q_row_stride=row,
                     stream=stream)


def ceil_div(a, b):
    return -(-a // b)


__all__ = ["RopeCache", "KVCache", "apply_rope", "apply_flash_decoding", "decode_step",
           "decode_step_unfused",
           "sm_scale", "BLOCK_SIZE"]
