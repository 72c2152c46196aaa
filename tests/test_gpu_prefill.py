"""HIP causal prefill (RoPE + cache write + MFMA attention of packed prompts)
vs the oracle, through the C ABI.  Roped q/k (in place) and the cache are
compared bit for bit; attention outputs within the stated tolerance
(max-abs 2e-3 fp16, 1e-2 bf16)."""
import numpy as np
import pytest
import torch

from lucciola_rs_amd import workloads as wl
from lucciola_rs_amd.engine import sm_scale
from gpu_util import TOL, from_dev, max_abs, rope_cache, say, to_dev, ulp_gate

pytestmark = pytest.mark.gpu


def biases(cfg, seed):
    rng = np.random.default_rng(seed)
    d = cfg.head_dim
    return (wl.to_bits(wl.normal(rng, (cfg.hq * d,), 0.5), cfg.dtype),
            wl.to_bits(wl.normal(rng, (cfg.hkv * d,), 0.5), cfg.dtype),
            wl.to_bits(wl.normal(rng, (cfg.hkv * d,), 0.5), cfg.dtype))


def gpu_prefill(luc, h: wl.HostPrefill, layer=0, max_ctx=None, bias=None):
    cfg = h.cfg
    d = cfg.head_dim
    rope = rope_cache(luc, d)
    qkv = to_dev(h.qkv, cfg.dtype)
    kp, vp = to_dev(h.k_pool, cfg.dtype), to_dev(h.v_pool, cfg.dtype)
    tables = torch.from_numpy(h.tables).cuda()
    cu = torch.from_numpy(h.cu_seqlens).cuda()
    sp = torch.from_numpy(h.start_pos).cuda()
    total = int(h.cu_seqlens[-1])
    out = torch.full((total, cfg.hq * d), 7.0, dtype=cfg.torch_dtype, device="cuda")
    qb, kb, vb = (None, None, None) if bias is None else (to_dev(x, cfg.dtype) for x in bias)
    max_ctx = h.max_ctx if max_ctx is None else max_ctx
    say(f"  [gpu] paged_prefill {cfg.name} rows={np.diff(h.cu_seqlens).tolist()[:8]} "
        f"starts={h.start_pos.tolist()[:8]} hq={cfg.hq} hkv={cfg.hkv} d={d} {cfg.dtype} "
        f"max_ctx={max_ctx} layer={layer} bias={bias is not None}")
    luc.paged_prefill(qkv, qb, kb, vb, rope.cos, rope.sin, kp, vp, tables, cu, sp, total, max_ctx,
                      layer, h.num_layers, cfg.hq, cfg.hkv, d, sm_scale(d), out)
    torch.cuda.synchronize()
    return dict(out=from_dev(out).reshape(total, cfg.hq, d), qkv=from_dev(qkv),
                k_pool=from_dev(kp), v_pool=from_dev(vp))


def oracle_prefill(orc, luc, h: wl.HostPrefill, layer=0, bias=None):
    cfg = h.cfg
    rope = rope_cache(luc, cfg.head_dim)
    cos, sin = rope.cos.cpu().numpy(), rope.sin.cpu().numpy()
    qkv, kp, vp = h.qkv.copy(), h.k_pool.copy(), h.v_pool.copy()
    qb, kb, vb = (None, None, None) if bias is None else bias
    out = orc.prefill(qkv, qb, kb, vb, cos, sin, kp, vp, h.tables, h.cu_seqlens, h.start_pos,
                      layer, cfg.hq, cfg.hkv, cfg.head_dim, sm_scale(cfg.head_dim), 16,
                      h.num_layers, cfg.dtype)
    return dict(out=out, qkv=qkv, k_pool=kp, v_pool=vp)


def assert_prefill_matches(orc, got, want, dtype, max_frac=0.5):
    """Bit-exact roped q/k and cache; attention outputs within the stated
    max-abs tolerance and within 4 storage units of the oracle's at the row's
    scale (ulp_gate: measured at most ~2.5), with at most `max_frac` of the
    elements differing at all (measured 18-43%)."""
    assert np.array_equal(got["qkv"], want["qkv"]), "RoPE'd q/k differ"
    assert np.array_equal(got["k_pool"], want["k_pool"]), "K pool differs"
    assert np.array_equal(got["v_pool"], want["v_pool"]), "V pool differs"
    o = orc.to_f32(got["out"], dtype)
    assert np.all(np.isfinite(o)), "non-finite attention output"
    err = max_abs(orc, got["out"], want["out"], dtype)
    say(f"  max|hip - oracle| = {err:.3e} (tol {TOL[dtype]})")
    assert err <= TOL[dtype]
    ulp_gate(orc, got["out"], want["out"], dtype, max_ulps=4, max_frac=max_frac)


SHAPES = [(14, 2, 64), (12, 2, 128), (28, 4, 128)]


@pytest.mark.parametrize("hq,hkv,d", SHAPES, ids=[f"{a}q{b}kv-d{c}" for a, b, c in SHAPES])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_prefill_ragged_prompts_and_prefixes(orc, luc, hq, hkv, d, dtype):
    """Prompts of 37, 64 and 1 rows after cached prefixes of 0, 5 and 130
    tokens (partial pages, a tile boundary, a one-row prompt)."""
    cfg = wl.PrefillConfig("ragged", 3, 0, hq, hkv, d, dtype, 0, 0, 0.5)
    h = wl.host_prefill_inputs(cfg, seed=7, rows=[37, 64, 1], starts=[0, 5, 130])
    assert_prefill_matches(orc, gpu_prefill(luc, h), oracle_prefill(orc, luc, h), dtype)


@pytest.mark.parametrize("group", [1, 2, 3, 4, 5, 6, 7, 8])
def test_prefill_every_group_size(orc, luc, group):
    cfg = wl.PrefillConfig(f"g{group}", 2, 0, 2 * group, 2, 64, "bf16", 0, 0, 0.5)
    h = wl.host_prefill_inputs(cfg, seed=group, rows=[70, 33], starts=[17, 64])
    assert_prefill_matches(orc, gpu_prefill(luc, h), oracle_prefill(orc, luc, h), "bf16")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_prefill_with_biases_and_layer(orc, luc, dtype):
    """q/k/v biases (Qwen2 has them) and a non-zero layer of a 3-layer cache."""
    cfg = wl.PrefillConfig("bias", 2, 0, 14, 2, 64, dtype, 0, 0, 0.5)
    h = wl.host_prefill_inputs(cfg, seed=11, num_layers=3, rows=[100, 29], starts=[3, 200])
    bias = biases(cfg, 12)
    for layer in (0, 2):
        assert_prefill_matches(orc, gpu_prefill(luc, h, layer=layer, bias=bias),
                               oracle_prefill(orc, luc, h, layer=layer, bias=bias), dtype)


@pytest.mark.parametrize("batch", [16, 17, 24])
def test_prefill_many_prompts(orc, luc, batch):
    """Many short ragged prompts, empty ones among them (the first, one in the
    middle and the last): the append kernel's workgroups straddle several
    sequences and its cu_seqlens search skips empty ones."""
    rng = np.random.default_rng(batch)
    rows = rng.integers(1, 40, batch)
    rows[[0, batch // 2, batch - 1]] = 0
    starts = rng.integers(0, 50, batch)
    cfg = wl.PrefillConfig(f"many{batch}", batch, 0, 14, 2, 64, "bf16", 0, 0, 0.5)
    h = wl.host_prefill_inputs(cfg, seed=batch, rows=rows, starts=starts)
    assert_prefill_matches(orc, gpu_prefill(luc, h), oracle_prefill(orc, luc, h), "bf16")


def test_prefill_4x2048_full(orc, luc):
    """The full prefill shape: 4 prompts x 2048 rows from an empty cache,
    14q/2kv, d=64, bf16, 128 pages per sequence."""
    cfg = wl.PREFILL_CONFIGS["prefill_4x2048"]
    h = wl.host_prefill_inputs(cfg, seed=2048)
    assert_prefill_matches(orc, gpu_prefill(luc, h), oracle_prefill(orc, luc, h), "bf16")


def test_prefill_matches_decode_steps(orc, luc):
    """Prefill of a prompt equals decoding its rows one at a time (the
    reference's own loop): the last row's output and the cache agree with the
    decode path's, within f32 rounding of the two accumulation orders."""
    from lucciola_rs_amd.engine import decode_step
    cfg = wl.PrefillConfig("vs_decode", 1, 0, 14, 2, 64, "bf16", 0, 0, 0.5)
    h = wl.host_prefill_inputs(cfg, seed=3, rows=[96], starts=[40], poison=False)
    got = gpu_prefill(luc, h)
    rope = rope_cache(luc, 64)
    kp, vp = to_dev(h.k_pool, "bf16"), to_dev(h.v_pool, "bf16")
    tables = torch.from_numpy(h.tables).cuda()
    row = cfg.row
    outs = []
    for i in range(96):
        qkv = to_dev(h.qkv[i: i + 1], "bf16")
        pos = torch.tensor([40 + i], dtype=torch.int32, device="cuda")
        out = torch.empty((1, 14 * 64), dtype=torch.bfloat16, device="cuda")
        ws = luc.workspace(1, 14, 2, 64, 40 + i + 1)
        decode_step(qkv, None, None, None, rope, kp, vp, tables, pos, 40 + i + 1, 0, 1, 14, 2, 64,
                    out, ws, 0, lib=luc)
        outs.append(out)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(kp), got["k_pool"]) and np.array_equal(from_dev(vp), got["v_pool"])
    dec = np.stack([orc.to_f32(from_dev(o).reshape(14, 64), "bf16") for o in outs])
    pre = orc.to_f32(got["out"], "bf16")
    err = float(np.max(np.abs(dec - pre)))
    say(f"  max|prefill - decode loop| = {err:.3e}")
    assert err <= TOL["bf16"]


def test_prefill_beyond_max_ctx_gives_nan(orc, luc):
    """A sequence whose prompt runs past the host bound max_ctx is flagged
    with NaN outputs; the others are computed normally.  RoPE and the cache
    write still cover every row the table can hold, flagged or not."""
    cfg = wl.PrefillConfig("over", 2, 0, 14, 2, 64, "bf16", 0, 0, 0.5)
    h = wl.host_prefill_inputs(cfg, seed=5, rows=[50, 20], starts=[0, 100])
    got = gpu_prefill(luc, h, max_ctx=60)  # sequence 1 reaches position 119
    o = orc.to_f32(got["out"], "bf16")
    assert np.all(np.isfinite(o[:50])) and np.all(np.isnan(o[50:]))
    want = oracle_prefill(orc, luc, h)
    assert np.array_equal(got["qkv"], want["qkv"]), "RoPE'd q/k differ"
    assert np.array_equal(got["k_pool"], want["k_pool"]) and np.array_equal(got["v_pool"], want["v_pool"])


def test_prefill_long_prompt_beyond_max_ctx_all_flagged(orc, luc):
    """A flagged prompt longer than the grid's tiles (130 rows against a bound
    of 40) has every one of its rows flagged; the other sequence matches the
    oracle."""
    cfg = wl.PrefillConfig("over_long", 2, 0, 14, 2, 64, "bf16", 0, 0, 0.5)
    h = wl.host_prefill_inputs(cfg, seed=6, rows=[30, 130], starts=[4, 0])
    got = gpu_prefill(luc, h, max_ctx=40)
    o = orc.to_f32(got["out"], "bf16")
    assert np.all(np.isnan(o[30:]))
    want = oracle_prefill(orc, luc, h)
    assert np.array_equal(got["qkv"], want["qkv"]), "RoPE'd q/k differ"
    assert np.array_equal(got["k_pool"], want["k_pool"]) and np.array_equal(got["v_pool"], want["v_pool"])
    err = float(np.max(np.abs(o[:30] - orc.to_f32(want["out"], "bf16")[:30])))
    assert err <= TOL["bf16"]
