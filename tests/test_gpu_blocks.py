"""A multi-sequence decode loop over the native page allocator (PagedKVCache):
sequences start, grow a page at a time, finish and release their pages, and
new sequences take the freed pages -- each step one luc_decode_step over the
live sequences, in lockstep with the oracle on the same tables.  Cache slots
bit-exact, attention outputs within the stated tolerance."""
import numpy as np
import pytest
import torch

from lucciola_rs_amd import workloads as wl
from lucciola_rs_amd.engine import PagedKVCache, decode_step, sm_scale
from gpu_util import TOL, from_dev, max_abs, rope_cache, say, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_decode_loop_with_admission_and_release(orc, luc, dtype):
    hq, hkv, d, slots, pool_pages, steps = 14, 2, 64, 6, 64, 90
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    rng = np.random.default_rng(41)
    cache = PagedKVCache(1, hkv, d, pool_pages, slots, 512, dtype=tdt)
    k_ref = np.zeros(tuple(cache.k_pool.shape), np.uint16)
    v_ref = np.zeros_like(k_ref)
    rope = rope_cache(luc, d)
    cos, sin = rope.cos.cpu().numpy(), rope.sin.cpu().numpy()
    length = np.zeros(slots, np.int64)          # tokens so far (-1: slot empty)
    target = rng.integers(10, 120, size=slots)  # tokens at which a sequence ends
    row = (hq + 2 * hkv) * d
    ws = luc.workspace(slots, hq, hkv, d, 512, 64)  # 64-token splits: split-K from 65 tokens
    admitted = finished = 0
    for step in range(steps):
        live = np.flatnonzero(length >= 0)
        cache.reserve_batch(live, length[live] + 1)
        cache.sync()
        tables = cache.blocks.table()[live]
        pos = length[live].astype(np.int32)
        qkv = wl.to_bits(rng.standard_normal((live.size, row)).astype(np.float32) * 0.5, dtype)
        q_dev = to_dev(qkv, dtype)
        out = torch.empty(live.size, hq * d, dtype=tdt, device="cuda")
        if step % 30 == 0:
            say(f"  [gpu] paged loop {dtype} step {step}: live {live.size}, free pages "
                f"{cache.blocks.num_free}")
        decode_step(q_dev, None, None, None, rope, cache.k_pool, cache.v_pool,
                    torch.from_numpy(tables).cuda(), torch.from_numpy(pos).cuda(),
                    int(pos.max()) + 1, 0, 1, hq, hkv, d, out, ws, split_tokens=64, lib=luc)
        want = orc.decode_step(qkv, None, None, None, cos, sin, k_ref, v_ref, tables, pos, 0, hq, hkv,
                               d, sm_scale(d), 16, 1, dtype)
        torch.cuda.synchronize()
        assert max_abs(orc, from_dev(out).reshape(want.shape), want, dtype) <= TOL[dtype], f"step {step}"
        assert np.array_equal(from_dev(q_dev), qkv), f"step {step}: roped q/k differ"
        length[live] += 1
        for s in live:  # finished sequences give their pages back; a new one takes the slot
            if length[s] >= target[s]:
                cache.release(int(s))
                finished += 1
                length[s], target[s] = 0, rng.integers(10, 120)
                admitted += 1
    assert np.array_equal(from_dev(cache.k_pool), k_ref) and np.array_equal(from_dev(cache.v_pool), v_ref)
    say(f"  {finished} sequences finished and {admitted} admitted over {steps} steps")
    assert finished >= 3
