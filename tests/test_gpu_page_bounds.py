"""Page ids outside [0, num_blocks): never used as an address.

The reference reads block-table entries unchecked (src/kernels/kv_cache.cu:28,
src/kernels/attention.cu:82); this library takes the pool size and treats an
entry outside it like a position outside the table row: no cache write, and
NaN for every attention output whose context reaches that page.  Each pool
here has SPARE pages past num_blocks filled with a sentinel and the bad
entries point into the spares (or are negative), so even a broken guard only
touches memory the test owns; the test then requires the spares untouched,
the pool unchanged except for the writes through valid pages, NaN where the
context reaches a bad page, and the oracle's results everywhere else."""
import numpy as np
import pytest
import torch

from lucciola_rs_amd import workloads as wl
from lucciola_rs_amd.engine import sm_scale
from gpu_util import TOL, from_dev, max_abs, oracle_step, rope_cache, say, to_dev

pytestmark = pytest.mark.gpu

SPARE = 4
SENTINEL = 0x3c01  # fp16 1.0009765625, bf16 a small positive number: never NaN


def _inputs(dtype, head_dim, hq, hkv, seed):
    cfg = wl.DecodeConfig(f"bounds_d{head_dim}", 4, hq, hkv, head_dim, dtype, 300, 900,
                          4 * 57 + 1, 0.5)
    h = wl.host_decode_inputs(cfg, seed=seed, poison=False)
    nb = h.k_pool.shape[0]  # real pages (the last one is the reserved page)
    spare = np.full((SPARE,) + h.k_pool.shape[1:], SENTINEL, np.uint16)
    k_pool = np.concatenate([h.k_pool, spare])
    v_pool = np.concatenate([h.v_pool, spare])
    tables = h.tables.copy()
    # sequence 0: a page in the middle of its context points into the spares;
    # sequence 1: a negative entry; sequence 2: the new token's page is the
    # first spare; sequence 3: untouched
    tables[0, (h.ctx[0] - 1) // 32] = nb + 1
    tables[1, 2] = -1
    tables[2, (h.ctx[2] - 1) // 16] = nb
    return cfg, h, nb, wl.HostDecode(cfg, 1, h.ctx, h.positions, tables, h.qkv, k_pool, v_pool)


def _pool_changes(before, after):
    """(page, layer, kv head, slot) of every changed cache row."""
    return {tuple(x) for x in np.argwhere(np.any(before != after, axis=-1))}


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "unfused"])
@pytest.mark.parametrize("head_dim,dtype,hq,hkv", [(64, "f16", 14, 2), (128, "bf16", 12, 2)])
@pytest.mark.parametrize("split", [0, 256, 384, 512, 1024])
def test_decode_never_uses_a_page_outside_the_pool(orc, luc, head_dim, dtype, hq, hkv, split, fused):
    """split 0 and 512 run the single-tile kernels at head_dim 64 (512 tokens =
    8 tiles of 64), 256 and 384 the 4-wave tile-pair kernels and 1024 the
    8-wave ones; at head_dim 128, 0 and 256 run the single-tile kernels (8
    tiles of 32), 384 the 4-wave tile-pair kernels and 512 and 1024 the
    8-wave ones (a multiple of 8 waves' tiles, one round of workgroups).
    Every sequence's q and k of the new token are roped in place, also where
    the new token's page lies outside the pool (only the cache write is
    skipped), on the fused and the unfused path alike."""
    cfg, clean, nb, h = _inputs(dtype, head_dim, hq, hkv, seed=head_dim + split)
    rope = rope_cache(luc, head_dim)
    qkv, kp, vp = to_dev(h.qkv, dtype), to_dev(h.k_pool, dtype), to_dev(h.v_pool, dtype)
    tables = torch.from_numpy(h.tables).cuda()
    pos = torch.from_numpy(h.positions).cuda()
    max_ctx = int(h.ctx.max())
    out = torch.zeros((cfg.batch, hq * head_dim), dtype=cfg.torch_dtype, device="cuda")
    ws = luc.workspace(cfg.batch, hq, hkv, head_dim, max_ctx, split)
    say(f"  [gpu] page bounds: d={head_dim} {dtype} split={split} {'fused' if fused else 'unfused'}"
        f" num_blocks={nb} (+{SPARE} spare pages)")
    common = dict(num_blocks=nb)
    if fused:
        luc.decode_step(qkv, None, None, None, rope.cos, rope.sin, kp, vp, tables, pos, cfg.batch,
                        max_ctx, 0, 1, hq, hkv, head_dim, sm_scale(head_dim), out, ws,
                        split_tokens=split, **common)
    else:
        luc.rope_append(qkv, None, qkv[:, hq * head_dim:], None, qkv[:, (hq + hkv) * head_dim:],
                        None, cfg.row, rope.cos, rope.sin, pos, tables, kp, vp, cfg.batch, 0, 1, hq,
                        hkv, head_dim, **common)
        luc.paged_decode(out, qkv, kp, vp, tables, pos, cfg.batch, max_ctx, 0, 1, hq, hkv, head_dim,
                         sm_scale(head_dim), split, ws, q_row_stride=cfg.row, **common)
    torch.cuda.synchronize()
    k_after, v_after = from_dev(kp), from_dev(vp)
    o = orc.to_f32(from_dev(out), dtype).reshape(cfg.batch, hq, head_dim)
    # the spares are untouched, and the only cache rows written are the new
    # tokens' slots of sequences 0, 1 and 3 (through valid pages)
    assert np.all(k_after[nb:] == SENTINEL) and np.all(v_after[nb:] == SENTINEL)
    want_rows = set()
    for b in (0, 1, 3):
        p = int(h.positions[b])
        want_rows |= {(int(h.tables[b, p // 16]), 0, kv, p % 16) for kv in range(hkv)}
    assert _pool_changes(h.k_pool, k_after) <= want_rows
    assert _pool_changes(h.v_pool, v_after) <= want_rows
    # (sequence 2's new token is written nowhere: its page is outside the pool)
    # NaN where the context reaches a bad page: sequences 0, 1 (all heads) and
    # 2 (its newest token's page)
    for b in (0, 1, 2):
        assert np.all(np.isnan(o[b])), f"sequence {b}"
    # q and k of every new token are roped in place, the bad pages'
    # sequences included (RoPE does not depend on the table)
    want_all = oracle_step(orc, luc, clean)
    assert np.array_equal(from_dev(qkv), want_all["qkv"]), "roped q/k rows differ"
    # sequence 3 as the oracle computes it on its own
    one = wl.HostDecode(wl.replace(cfg, batch=1), 1, clean.ctx[3:4], clean.positions[3:4],
                        clean.tables[3:4], clean.qkv[3:4], clean.k_pool, clean.v_pool)
    want = oracle_step(orc, luc, one)
    err = max_abs(orc, from_dev(out)[3:4], want["out"].reshape(1, -1), dtype)
    say(f"  valid sequence: max|hip - oracle| = {err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("head_dim", [64, 128])
def test_prefill_never_uses_a_page_outside_the_pool(orc, luc, head_dim):
    """Two prompts of 200 rows after cached prefixes of 40 and 0 rows: the
    first has table page 7 (tokens 112..127) outside the pool, the second
    page 3 negative.  Rows before the bad page match the oracle; rows at or
    after it are NaN; no cache row is written through the bad page and the
    spares are untouched."""
    hq, hkv, dtype = (14, 2, "bf16") if head_dim == 64 else (12, 2, "bf16")
    cfg = wl.PrefillConfig(f"pb{head_dim}", 2, 200, hq, hkv, head_dim, dtype, 0, 0, 0.5)
    h = wl.host_prefill_inputs(cfg, seed=5, poison=False, rows=np.array([200, 200]),
                               starts=np.array([40, 0]))
    nb = h.k_pool.shape[0]
    spare = np.full((SPARE,) + h.k_pool.shape[1:], SENTINEL, np.uint16)
    k_pool = np.concatenate([h.k_pool, spare])
    v_pool = np.concatenate([h.v_pool, spare])
    tables = h.tables.copy()
    tables[0, 7] = nb + 2
    tables[1, 3] = -5
    rope = rope_cache(luc, head_dim)
    qkv = to_dev(h.qkv, dtype)
    kp, vp = to_dev(k_pool, dtype), to_dev(v_pool, dtype)
    total = int(h.cu_seqlens[-1])
    out = torch.zeros((total, hq * head_dim), dtype=torch.bfloat16, device="cuda")
    say(f"  [gpu] prefill page bounds d={head_dim} num_blocks={nb} (+{SPARE} spare)")
    luc.paged_prefill(qkv, None, None, None, rope.cos, rope.sin, kp, vp,
                      torch.from_numpy(tables).cuda(), torch.from_numpy(h.cu_seqlens).cuda(),
                      torch.from_numpy(h.start_pos).cuda(), total, h.max_ctx, 0, 1, hq, hkv,
                      head_dim, sm_scale(head_dim), out, num_blocks=nb)
    torch.cuda.synchronize()
    k_after, v_after = from_dev(kp), from_dev(vp)
    assert np.all(k_after[nb:] == SENTINEL) and np.all(v_after[nb:] == SENTINEL)
    # the oracle on the valid table (bad entries replaced by their real pages)
    cos, sin = rope.cos.cpu().numpy(), rope.sin.cpu().numpy()
    q_o, kp_o, vp_o = h.qkv.copy(), h.k_pool.copy(), h.v_pool.copy()
    want = orc.prefill(q_o, None, None, None, cos, sin, kp_o, vp_o, h.tables, h.cu_seqlens,
                       h.start_pos, 0, hq, hkv, head_dim, sm_scale(head_dim), 16, 1, dtype)
    got = orc.to_f32(from_dev(out), dtype).reshape(total, hq, head_dim)
    for b, bad_page in ((0, 7), (1, 3)):
        r0, r1 = int(h.cu_seqlens[b]), int(h.cu_seqlens[b + 1])
        pos = int(h.start_pos[b]) + np.arange(r1 - r0)
        ok = pos < bad_page * 16
        assert np.all(np.isnan(got[r0:r1][~ok])), f"sequence {b}: rows past the bad page"
        good = want[r0:r1][ok]
        err = float(np.max(np.abs(got[r0:r1][ok] - orc.to_f32(good, dtype))))
        say(f"  sequence {b}: {ok.sum()} rows before page {bad_page}: max err {err:.3e}")
        assert err <= TOL[dtype]
    # no cache row of a bad page's tokens was written (the rest as the oracle)
    for b, bad_page in ((0, 7), (1, 3)):
        real = int(h.tables[b, bad_page])
        assert np.array_equal(k_after[real], h.k_pool[real]), "write through a bad entry"
