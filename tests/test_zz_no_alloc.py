"""luc_decode_step_noalloc (the library's fixed per-device scratch as the
split-K workspace) against luc_decode_step with a caller workspace, through
the C ABI: two calls in a row, the second with a smaller batch and context,
then the first again.  The two entry points run the same kernels on the same
split plan, so every output is compared bit for bit: roped q/k in the qkv
rows, both pools and the attention output."""
import numpy as np
import pytest
import torch

from lucciola_rs_amd import library
from lucciola_rs_amd import workloads as wl
from lucciola_rs_amd.engine import sm_scale
from gpu_util import from_dev, rope_cache, say, to_dev

pytestmark = pytest.mark.gpu


def _inputs(batch, lo, hi, seed):
    cfg = wl.scaled(wl.CONFIGS["batch32_mixed"], batch=batch, ctx_lo=lo, ctx_hi=hi,
                    pool_pages=batch * ((hi + 15) // 16) + 3)
    h = wl.host_decode_inputs(cfg, seed=seed, num_layers=2)
    rng = np.random.default_rng(seed + 1)
    d = cfg.head_dim
    bias = wl.to_bits(rng.standard_normal(cfg.row) * 0.1, cfg.dtype)
    return h, bias


def _run(luc, h, bias, split, noalloc):
    cfg = h.cfg
    d = cfg.head_dim
    rope = rope_cache(luc, d)
    qkv, kp, vp = to_dev(h.qkv, cfg.dtype), to_dev(h.k_pool, cfg.dtype), to_dev(h.v_pool, cfg.dtype)
    b = to_dev(bias, cfg.dtype)
    qb, kb, vb = b[:cfg.hq * d], b[cfg.hq * d:(cfg.hq + cfg.hkv) * d], b[(cfg.hq + cfg.hkv) * d:]
    tables = torch.from_numpy(h.tables).cuda()
    pos = torch.from_numpy(h.positions).cuda()
    max_ctx = int(h.ctx.max())
    out = torch.full((cfg.batch, cfg.hq * d), 7.0, dtype=cfg.torch_dtype, device="cuda")
    say(f"  [gpu] decode_step{'_noalloc' if noalloc else ''} B={cfg.batch} max_ctx={max_ctx} "
        f"split={split} layer=1")
    common = (qkv, qb, kb, vb, rope.cos, rope.sin, kp, vp, tables, pos, cfg.batch, max_ctx, 1,
              h.num_layers, cfg.hq, cfg.hkv, d, sm_scale(d))
    if noalloc:
        luc.decode_step_noalloc(*common, out, split_tokens=split, qkv_row_stride=cfg.row)
    else:
        ws = luc.workspace(cfg.batch, cfg.hq, cfg.hkv, d, max_ctx, split)
        luc.decode_step(*common, out, ws, split, qkv_row_stride=cfg.row)
    torch.cuda.synchronize()
    return {"out": from_dev(out), "qkv": from_dev(qkv), "k_pool": from_dev(kp),
            "v_pool": from_dev(vp)}


def _same(a, b):
    for k in ("out", "qkv", "k_pool", "v_pool"):
        assert np.array_equal(a[k], b[k]), f"{k} differs"


def test_noalloc_matches_decode_step_twice(luc):
    big, big_bias = _inputs(6, 300, 3000, seed=61)
    small, small_bias = _inputs(3, 50, 700, seed=62)
    # the second call is smaller: fewer sequences and splits, so the scratch
    # still holds the first call's partials past what the second one uses
    first = _run(luc, big, big_bias, 64, noalloc=True)
    _same(first, _run(luc, big, big_bias, 64, noalloc=False))
    second = _run(luc, small, small_bias, 64, noalloc=True)
    _same(second, _run(luc, small, small_bias, 64, noalloc=False))
    # the library's automatic split choice, and the first input once more
    _same(_run(luc, small, small_bias, 0, noalloc=True), _run(luc, small, small_bias, 0, noalloc=False))
    _same(_run(luc, big, big_bias, 64, noalloc=True), first)


def test_noalloc_rejects_sizes_beyond_the_scratch(luc):
    """64 sequences of 28q/4kv, d=128 at max_ctx 16384 in 64-token splits need
    far more than the fixed scratch: a clear error before any launch."""
    need = luc.workspace_size(64, 28, 4, 128, 16384, 64)
    assert need > 16 << 20
    out = torch.full((64, 28 * 128), 3.0, dtype=torch.bfloat16, device="cuda")
    qkv = torch.zeros((64, 36 * 128), dtype=torch.bfloat16, device="cuda")
    pool = torch.zeros((8, 1, 4, 16, 128), dtype=torch.bfloat16, device="cuda")
    tables = torch.zeros((64, 1024), dtype=torch.int32, device="cuda")
    pos = torch.zeros(64, dtype=torch.int32, device="cuda")
    rope = rope_cache(luc, 128)
    with pytest.raises(library.LucError) as e:
        luc.decode_step_noalloc(qkv, None, None, None, rope.cos, rope.sin, pool, pool, tables, pos,
                                64, 16384, 0, 1, 28, 4, 128, sm_scale(128), out, split_tokens=64)
    assert e.value.code == -5 and "scratch" in str(e.value)
    torch.cuda.synchronize()
    assert bool(torch.all(out == 3.0))
