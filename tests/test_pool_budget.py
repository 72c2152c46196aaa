"""KV pool sizing from the VRAM budget, as KVCache::new does it
(src/layers/kv_cache.rs:37-59), and its failure path (kv_cache.rs:40-48):
engine.pool_blocks on synthetic (free, total) pairs, no GPU."""
import numpy as np
import pytest

from lucciola_rs_amd.engine import KVCache, pool_blocks

GIB = 1 << 30
# Qwen2.5-0.5B: 24 layers, 2 kv heads, head_dim 64 -> K and V of 16 tokens in bf16
PAGE_BYTES = 2 * 24 * 2 * 16 * 64 * 2


def test_page_bytes_and_the_max_position_cap():
    assert PAGE_BYTES == 196608
    # 288 GiB card, 8 GiB in use, fraction 0.9: far more than the 2048 pages
    # that 32768 positions need
    assert pool_blocks(280 * GIB, 288 * GIB, 0.9, 24, 2, 64, 32768) == 2048


def test_budget_is_an_f32_product_less_the_used_memory():
    free, total, frac = 7 * GIB + 12345, 8 * GIB, 0.3
    used = total - free
    budget = int(np.float32(total) * np.float32(frac)) - used  # (total as f32 * fraction) as usize
    want = budget // PAGE_BYTES
    assert want < 2048 * 64
    assert pool_blocks(free, total, frac, 24, 2, 64, 2048 * 16 * 64) == want
    # the f32 product is not the f64 one at this size
    assert int(np.float32(total) * np.float32(frac)) != int(total * frac)


def test_budget_below_the_used_memory_fails_with_the_reference_message():
    with pytest.raises(RuntimeError, match="Not enough available GPU memory for KV Cache allocation"):
        pool_blocks(1 * GIB, 8 * GIB, 0.5, 24, 2, 64, 32768)  # 7 GiB used > 4 GiB budget
    with pytest.raises(RuntimeError, match="requested fraction: 0.5"):
        KVCache.from_budget(24, 2, 64, 32768, 0.5, mem_info=(1 * GIB, 8 * GIB), device="cpu")


def test_budget_just_above_the_used_memory_gives_what_fits():
    free, total = 6 * GIB, 8 * GIB  # 2 GiB used
    frac = 0.25 + 3 * PAGE_BYTES / (8 * GIB)  # a budget of 2 GiB + 3 pages (up to f32 rounding)
    got = pool_blocks(free, total, frac, 24, 2, 64, 32768)
    assert got == (int(np.float32(total) * np.float32(frac)) - 2 * GIB) // PAGE_BYTES
    assert 2 <= got <= 3
    assert pool_blocks(free, total, 0.25, 24, 2, 64, 32768) == 0  # budget equals the used memory
