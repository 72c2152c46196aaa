"""HIP decode path (RoPE + paged append + split-K attention + combine) vs the
oracle, through the C ABI.  Integer/byte work (RoPE'd q and k, cache slots) is
compared bit for bit; attention outputs within the stated tolerance
(max-abs 2e-3 fp16, 1e-2 bf16)."""
import dataclasses

import numpy as np
import pytest
import torch

from lucciola_rs_amd import workloads as wl
from gpu_util import TOL, from_dev, gpu_step, max_abs, oracle_step, say

pytestmark = pytest.mark.gpu


def assert_step_matches(orc, got, want, dtype, gate=None):
    """Bit-exact cache and roped q/k; attention output within the stated
    tolerance and, where given, within `gate`: a regression bound at about
    ten times the error measured on the same inputs."""
    assert np.array_equal(got["qkv"], want["qkv"]), "RoPE'd q/k differ"
    assert np.array_equal(got["k_pool"], want["k_pool"]), "K pool differs"
    assert np.array_equal(got["v_pool"], want["v_pool"]), "V pool differs"
    o = orc.to_f32(got["out"], dtype)
    assert np.all(np.isfinite(o)), "non-finite attention output"
    err = max_abs(orc, got["out"], want["out"], dtype)
    say(f"  max|hip - oracle| = {err:.3e} (tol {TOL[dtype]}, gate {gate})")
    assert err <= TOL[dtype]
    if gate is not None:
        assert err <= gate


SMALL = [
    # (config, batch, ctx_lo, ctx_hi)
    ("batch32_mixed", 5, 1, 600),
    ("batch64_long", 4, 100, 1500),
    ("batch8_32k", 2, 700, 2100),
]


@pytest.mark.parametrize("name,batch,lo,hi", SMALL)
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("fused", [True, False], ids=["fused", "unfused"])
def test_decode_small_configs(orc, luc, name, batch, lo, hi, dtype, fused):
    cfg = wl.scaled(wl.CONFIGS[name], batch=batch, ctx_lo=lo, ctx_hi=hi,
                    pool_pages=batch * ((hi + 15) // 16) + 3)
    cfg = wl.replace(cfg, dtype=dtype)
    h = wl.host_decode_inputs(cfg, seed=11)
    assert_step_matches(orc, gpu_step(luc, h, fused=fused), oracle_step(orc, luc, h), dtype)


@pytest.mark.parametrize("group", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("dtype,kernel", [("bf16", "t1"), ("bf16", "t2"), ("f16", "t2"),
                                          ("bf16", "t2w8"), ("f16", "t2w8")])
def test_decode_every_group_size(orc, luc, group, head_dim, dtype, kernel):
    """Every group size on every kernel shape: the automatic split of these
    small batches runs the single-tile (_t1) kernels; 256-token splits at
    head_dim 64 and 384 at 128 the 4-wave tile-pair (_t2) kernels; 1024 at
    head_dim 64 and 512 at 128, a multiple of 8 waves' tiles in a launch of
    one round, the 8-wave ones (_t2w8).  Two tiles per wave; at head_dim 128
    the step variants and group size 8 keep PV on v_dot2.  Both dtypes."""
    hkv = 2
    hi = 2600 if (kernel, head_dim) == ("t2w8", 64) else 900  # several 1024-token splits
    cfg = wl.DecodeConfig(f"g{group}", 3, group * hkv, hkv, head_dim, dtype, 1, hi,
                          3 * (hi // 16 + 1) + 1, 0.5)
    h = wl.host_decode_inputs(cfg, seed=group)
    split = {"t1": 0, "t2": 256 if head_dim == 64 else 384,
             "t2w8": 1024 if head_dim == 64 else 512}[kernel]
    assert_step_matches(orc, gpu_step(luc, h, split_tokens=split), oracle_step(orc, luc, h), dtype)
    assert_step_matches(orc, gpu_step(luc, h, split_tokens=split, fused=False),
                        oracle_step(orc, luc, h), dtype)


def test_decode_layers_and_page_boundaries(orc, luc):
    # contexts at page boundaries, a non-zero layer of a 3-layer pool
    cfg = wl.DecodeConfig("bounds", 8, 14, 2, 64, "f16", 1, 1, 8 * 20, 0.5)
    h = wl.host_decode_inputs(cfg, seed=3, num_layers=3, poison=False)
    ctx = np.array([1, 15, 16, 17, 32, 33, 255, 257], np.int32)
    rng = np.random.default_rng(5)
    tables = np.full((8, 20), cfg.pool_pages, np.int32)
    perm = rng.permutation(cfg.pool_pages)
    off = 0
    for b, c in enumerate(ctx):
        n = (c + 15) // 16
        tables[b, :n] = perm[off: off + n]
        off += n
    h = wl.HostDecode(cfg, 3, ctx, ctx - 1, tables, h.qkv, h.k_pool, h.v_pool)
    for layer in (0, 2):
        assert_step_matches(orc, gpu_step(luc, h, layer=layer),
                            oracle_step(orc, luc, h, layer=layer), "f16")


def test_single_512(orc, luc):
    """Single sequence, 14q/2kv, d=64, fp16, ctx 512, permuted table."""
    cfg = wl.CONFIGS["single_512"]
    h = wl.host_decode_inputs(cfg, seed=2024)
    assert_step_matches(orc, gpu_step(luc, h), oracle_step(orc, luc, h), "f16")


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "unfused"])
def test_batch32_mixed_full(orc, luc, fused):
    """B=32, ctx U{128..4096}, pool 16384 pages, fp16 -- full size, one layer."""
    cfg = wl.CONFIGS["batch32_mixed"]
    h = wl.host_decode_inputs(cfg, seed=1)
    assert_step_matches(orc, gpu_step(luc, h, fused=fused), oracle_step(orc, luc, h), "f16",
                        gate=2e-4)  # measured 6.1e-5: one fp16 unit at these magnitudes


def test_batch8_32k_full(orc, luc):
    """B=8, ctx 32768 each, 12q/2kv d=128 bf16, 1% x8 outliers -- full size."""
    cfg = wl.CONFIGS["batch8_32k"]
    h = wl.host_decode_inputs(cfg, seed=8)
    assert_step_matches(orc, gpu_step(luc, h), oracle_step(orc, luc, h), "bf16",
                        gate=5e-4)  # measured 6.1e-5


@pytest.mark.parametrize("split", [0, 512], ids=["auto", "split512"])
def test_batch64_long_full(orc, luc, split):
    """B=64, ctx U{1024..16384}, 28q/4kv d=128 bf16 -- full size, one layer;
    automatic splits, and 512-token splits (2 to 32 per sequence, the
    configuration's split-K regime)."""
    cfg = wl.CONFIGS["batch64_long"]
    h = wl.host_decode_inputs(cfg, seed=64, poison=False)
    assert_step_matches(orc, gpu_step(luc, h, split_tokens=split), oracle_step(orc, luc, h), "bf16",
                        gate=1e-3)  # measured 1.2e-4


def bf16_units(a, b):
    """Distance in bf16 units in the last place between two bit arrays."""
    def key(x):
        x = x.astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7fff), x & 0x7fff)
    return np.abs(key(a) - key(b))


def test_split_count_independence(orc, luc):
    """The output does not depend on how the context is split: with every
    context at most 2048 tokens, 2048-token splits are one split per
    sequence (no merge); 128..1024-token splits (2 to 16 per sequence) give
    the same bf16 output to within one unit in the last place, on at most 1%
    of the outputs (f32 merge rounding crossing a bf16 rounding boundary)."""
    cfg = wl.scaled(wl.CONFIGS["batch8_32k"], batch=3, ctx_lo=1500, ctx_hi=2048,
                    pool_pages=3 * 128 + 1)
    h = wl.host_decode_inputs(cfg, seed=17)
    outs = {s: gpu_step(luc, h, split_tokens=s)["out"] for s in (128, 256, 512, 1024, 2048)}
    ref = outs[2048]  # one split per sequence
    want = oracle_step(orc, luc, h)["out"]
    say(f"  one split vs oracle: {max_abs(orc, ref, want, 'bf16'):.3e}")
    assert max_abs(orc, ref, want, "bf16") <= 2e-3  # measured 2.4e-4
    for s, o in outs.items():
        u = bf16_units(o, ref)
        say(f"  split {s}: max {u.max()} bf16 units from one split, {np.count_nonzero(u)} of {u.size} differ")
        assert u.max() <= 1 and np.count_nonzero(u) <= u.size // 100


@pytest.mark.parametrize("split", [64, 128, 192, 256, 512, 1024, 2048])
def test_split_sizes_fp16_against_oracle(orc, luc, split):
    """Every split size (one tile per split, tile pairs, and splits walking
    several pairs) matches the oracle at the fp16 tolerance, at the
    batch32_mixed shape with contexts up to 4096."""
    cfg = wl.scaled(wl.CONFIGS["batch32_mixed"], batch=6, ctx_lo=200, ctx_hi=4096,
                    pool_pages=6 * 256 + 1)
    h = wl.host_decode_inputs(cfg, seed=29)
    want = oracle_step(orc, luc, h)
    got = gpu_step(luc, h, split_tokens=split)
    assert_step_matches(orc, got, want, "f16")


def test_page_permutation_is_bit_exact(orc, luc):
    """Moving pages in the pool and remapping the table changes nothing."""
    cfg = wl.scaled(wl.CONFIGS["batch32_mixed"], batch=4, ctx_lo=200, ctx_hi=1200,
                    pool_pages=4 * 75 + 1)
    h = wl.host_decode_inputs(cfg, seed=23, poison=False)
    a = gpu_step(luc, h)["out"]
    perm = np.random.default_rng(0).permutation(h.k_pool.shape[0])
    inv = np.argsort(perm)
    h2 = wl.HostDecode(cfg, 1, h.ctx, h.positions, inv[h.tables].astype(np.int32),
                       h.qkv, h.k_pool[perm].copy(), h.v_pool[perm].copy())
    b = gpu_step(luc, h2)["out"]
    assert np.array_equal(a, b)


def test_gqa_group_with_equal_queries(orc, luc):
    """q-heads of one GQA group with equal q give equal outputs."""
    cfg = wl.scaled(wl.CONFIGS["batch32_mixed"], batch=2, ctx_lo=300, ctx_hi=900,
                    pool_pages=2 * 57 + 1)
    h = wl.host_decode_inputs(cfg, seed=31)
    qkv = h.qkv.copy()
    d = cfg.head_dim
    for hd in range(1, 7):  # heads 0..6 share kv head 0
        qkv[:, hd * d:(hd + 1) * d] = qkv[:, :d]
    h2 = wl.HostDecode(cfg, 1, h.ctx, h.positions, h.tables, qkv, h.k_pool, h.v_pool)
    out = gpu_step(luc, h2)["out"]
    for hd in range(1, 7):
        assert np.array_equal(out[:, hd], out[:, 0])


def test_empty_and_overlong_contexts_give_nan(orc, luc):
    """An empty context (position -1) is 0/0 as in the reference; a context
    longer than the host bound max_ctx is flagged with NaN, never truncated."""
    cfg = wl.scaled(wl.CONFIGS["batch32_mixed"], batch=3, ctx_lo=500, ctx_hi=500,
                    pool_pages=3 * 32 + 1)
    h = wl.host_decode_inputs(cfg, seed=41, poison=False)
    # sequence 1 empty: skip its append too by running decode only
    from gpu_util import rope_cache, to_dev
    from lucciola_rs_amd.engine import sm_scale
    kp, vp = to_dev(h.k_pool, "f16"), to_dev(h.v_pool, "f16")
    q = to_dev(h.qkv, "f16")
    tables = torch.from_numpy(h.tables).cuda()
    pos = torch.tensor([499, -1, 499], dtype=torch.int32, device="cuda")
    out = torch.zeros((3, cfg.hq * 64), dtype=torch.float16, device="cuda")
    ws = luc.workspace(3, 14, 2, 64, 300, 64)
    say("  [gpu] paged_decode max_ctx=300 < ctx=500, split 64")
    luc.paged_decode(out, q, kp, vp, tables, pos, 3, 300, 0, 1, 14, 2, 64, sm_scale(64), 64,
                     ws, q_row_stride=cfg.row)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    assert np.all(np.isnan(o)), "every sequence is empty or over max_ctx"
    ws = luc.workspace(3, 14, 2, 64, 500)
    out.zero_()
    say("  [gpu] paged_decode max_ctx=500")
    luc.paged_decode(out, q, kp, vp, tables, pos, 3, 500, 0, 1, 14, 2, 64, sm_scale(64), 0, ws,
                     q_row_stride=cfg.row)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    assert np.all(np.isnan(o[1])) and np.all(np.isfinite(o[[0, 2]]))


@pytest.mark.parametrize("name,dtype,split", [("batch64_long", "bf16", 512),
                                               ("batch32_mixed", "f16", 256)])
def test_longest_first_order_mixed_positions(orc, luc, name, dtype, split):
    """The tile-pair kernels with several splits per sequence take their work
    longest first: the full splits, then each sequence's partial last split by
    length.  A batch mixing contexts that end on a split edge, one token past
    it, one short of it, short and long ones, an empty context and one past
    max_ctx gives the oracle's output for every valid sequence and NaN for
    the others, on two calls in a row on one workspace (the arrival counters
    left at zero)."""
    S = split
    ctxs = [S, S + 1, 3 * S, 3 * S - 1, 17, 1, 2 * S + S // 2, 0, 5 * S + 4, 5 * S, S - 1, 4 * S + 7]
    max_ctx = 5 * S
    cfg = wl.scaled(wl.CONFIGS[name], batch=len(ctxs), ctx_lo=max_ctx + 8, ctx_hi=max_ctx + 8)
    cfg = dataclasses.replace(cfg, dtype=dtype)
    h = wl.host_decode_inputs(cfg, seed=77, poison=False)
    pos_np = np.array(ctxs, np.int32) - 1
    from gpu_util import to_dev
    from lucciola_rs_amd.engine import sm_scale
    q = to_dev(h.qkv, dtype)
    kp, vp = to_dev(h.k_pool, dtype), to_dev(h.v_pool, dtype)
    tables = torch.from_numpy(h.tables).cuda()
    pos = torch.from_numpy(pos_np).cuda()
    ws = luc.workspace(cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim, max_ctx, split)
    outs = []
    for call in range(2):
        out = torch.full((cfg.batch, cfg.hq * cfg.head_dim), 7.0, dtype=cfg.torch_dtype, device="cuda")
        say(f"  [gpu] paged_decode {name} B={cfg.batch} d={cfg.head_dim} {dtype} split {split} "
            f"max_ctx {max_ctx}, call {call}")
        luc.paged_decode(out, q, kp, vp, tables, pos, cfg.batch, max_ctx, 0, 1, cfg.hq, cfg.hkv,
                         cfg.head_dim, sm_scale(cfg.head_dim), split, ws, q_row_stride=cfg.row)
        torch.cuda.synchronize()
        outs.append(from_dev(out).reshape(cfg.batch, cfg.hq, cfg.head_dim))
    assert np.array_equal(outs[0], outs[1]), "the second call differs"
    o = orc.to_f32(outs[0], dtype)
    bad = [i for i, c in enumerate(ctxs) if c < 1 or c > max_ctx]
    good = [i for i in range(len(ctxs)) if i not in bad]
    assert np.all(np.isnan(o[bad])), "an empty or over-long context without NaN"
    want = orc.decode_batch(h.qkv[good], h.k_pool, h.v_pool, h.tables[good], pos_np[good], 0,
                            cfg.hq, cfg.hkv, cfg.head_dim, sm_scale(cfg.head_dim), 16, 1, dtype)
    assert np.all(np.isfinite(o[good]))
    err = max_abs(orc, outs[0][good], want, dtype)
    say(f"  max|hip - oracle| = {err:.3e} over the valid sequences (tol {TOL[dtype]})")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("batch", [1, 2, 37, 64, 65])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_longest_first_order_batch_sizes(orc, luc, batch, head_dim):
    """The tile-pair kernels' longest-first work order across batch sizes:
    one sequence per lane of the ordering wave up to 64, plain split-major
    order at 65.  Random contexts, a third of those of a split or more cut
    down to a multiple of the split (only full splits; a context is only
    ever shortened, so its pages stay allocated), the fused step and the
    unfused path alike."""
    hkv, group = 2, 7
    split = 256 if head_dim == 64 else 512
    hi = 6 * split
    cfg = wl.DecodeConfig(f"lf{batch}", batch, group * hkv, hkv, head_dim, "bf16", 1, hi,
                          batch * (hi // 16 + 1) + 1, 0.5)
    h = wl.host_decode_inputs(cfg, seed=batch * 7 + head_dim, poison=False)
    ctx = h.ctx.copy()
    cut = (np.arange(batch) % 3 == 1) & (ctx >= split)
    ctx[cut] = ctx[cut] // split * split
    h = dataclasses.replace(h, ctx=ctx, positions=(ctx - 1).astype(np.int32))
    want = oracle_step(orc, luc, h)
    # gate: two bf16 units at |x| < 0.5 (measured at most one)
    assert_step_matches(orc, gpu_step(luc, h, split_tokens=split), want, "bf16", gate=4e-3)
    assert_step_matches(orc, gpu_step(luc, h, split_tokens=split, fused=False), want, "bf16",
                        gate=4e-3)


def test_workspace_reuse_across_launches(orc, luc):
    """One workspace serves many launches (and layers) with identical results."""
    cfg = wl.scaled(wl.CONFIGS["batch32_mixed"], batch=6, ctx_lo=300, ctx_hi=3000,
                    pool_pages=6 * 188 + 1)
    h = wl.host_decode_inputs(cfg, seed=51, num_layers=2, poison=False)
    from gpu_util import to_dev
    from lucciola_rs_amd.engine import sm_scale
    kp, vp = to_dev(h.k_pool, "f16"), to_dev(h.v_pool, "f16")
    q = to_dev(h.qkv, "f16")
    tables = torch.from_numpy(h.tables).cuda()
    pos = torch.from_numpy(h.positions).cuda()
    max_ctx = int(h.ctx.max())
    ws = luc.workspace(6, 14, 2, 64, max_ctx, 256)
    outs = []
    say("  [gpu] paged_decode x8 on one workspace")
    for i in range(8):
        out = torch.zeros((6, 14 * 64), dtype=torch.float16, device="cuda")
        luc.paged_decode(out, q, kp, vp, tables, pos, 6, max_ctx, i % 2, 2, 14, 2, 64,
                         sm_scale(64), 256, ws, q_row_stride=cfg.row)
        outs.append(out)
    # a call with another batch and max_ctx on the same workspace in between
    # (the arrival counters keep their place), then the first call again
    small = torch.zeros((3, 14 * 64), dtype=torch.float16, device="cuda")
    small_ctx = int(h.ctx[:3].max())
    say(f"  [gpu] paged_decode batch 3, max_ctx {small_ctx} on the same workspace")
    luc.paged_decode(small, q[:3], kp, vp, tables[:3], pos[:3], 3, small_ctx, 0, 2, 14, 2, 64,
                     sm_scale(64), 128, ws, q_row_stride=cfg.row)
    again = torch.zeros((6, 14 * 64), dtype=torch.float16, device="cuda")
    luc.paged_decode(again, q, kp, vp, tables, pos, 6, max_ctx, 0, 2, 14, 2, 64,
                     sm_scale(64), 256, ws, q_row_stride=cfg.row)
    torch.cuda.synchronize()
    for i in range(2, 8):
        assert torch.equal(outs[i], outs[i % 2])
    assert not torch.equal(outs[0], outs[1])
    assert torch.equal(again, outs[0])
    assert max_abs(orc, from_dev(small), from_dev(outs[0][:3]), "f16") <= TOL["f16"]
