"""Helpers for the GPU parity tests: move bit patterns to/from the device and
run one decode step through the C ABI and through the oracle."""
from __future__ import annotations

import sys

import numpy as np
import torch

from lucciola_rs_amd import workloads as wl
from lucciola_rs_amd.engine import RopeCache, decode_step, decode_step_unfused, sm_scale

# tolerance on attention outputs (max-abs vs the reference algorithm)
TOL = {"f16": 2e-3, "bf16": 1e-2}


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def to_dev(bits, dtype):
    return wl.bits_to_tensor(np.ascontiguousarray(bits), dtype).cuda()


def from_dev(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


_ROPE = {}


def rope_cache(luc, head_dim, max_pos=32768, theta=1e6):
    key = (head_dim, max_pos, theta)
    if key not in _ROPE:
        _ROPE[key] = RopeCache(max_pos, head_dim, theta, lib=luc, device="cuda")
    return _ROPE[key]


def gpu_step(luc, h: wl.HostDecode, split_tokens=0, layer=0, max_ctx=None, positions=None,
             fused=True):
    """One decode step through the C ABI on fresh device copies of h: the fused
    single launch (luc_decode_step) or luc_rope_append + luc_paged_decode."""
    cfg = h.cfg
    rope = rope_cache(luc, cfg.head_dim)
    qkv = to_dev(h.qkv, cfg.dtype)
    kp = to_dev(h.k_pool, cfg.dtype)
    vp = to_dev(h.v_pool, cfg.dtype)
    tables = torch.from_numpy(h.tables).cuda()
    pos_np = h.positions if positions is None else positions
    pos = torch.from_numpy(np.ascontiguousarray(pos_np, dtype=np.int32)).cuda()
    max_ctx = int(h.ctx.max()) if max_ctx is None else max_ctx
    out = torch.full((cfg.batch, cfg.hq * cfg.head_dim), 7.0, dtype=cfg.torch_dtype,
                     device="cuda")
    ws = luc.workspace(cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim, max_ctx, split_tokens)
    say(f"  [gpu] decode_step{'' if fused else '_unfused'} {cfg.name} B={cfg.batch} hq={cfg.hq} "
        f"hkv={cfg.hkv} d={cfg.head_dim} {cfg.dtype} max_ctx={max_ctx} split={split_tokens} "
        f"layer={layer}")
    fn = decode_step if fused else decode_step_unfused
    fn(qkv, None, None, None, rope, kp, vp, tables, pos, max_ctx, layer, h.num_layers,
       cfg.hq, cfg.hkv, cfg.head_dim, out, ws, split_tokens, lib=luc)
    torch.cuda.synchronize()
    return dict(out=from_dev(out).reshape(cfg.batch, cfg.hq, cfg.head_dim), qkv=from_dev(qkv),
                k_pool=from_dev(kp), v_pool=from_dev(vp))


def oracle_step(orc, luc, h: wl.HostDecode, layer=0):
    cfg = h.cfg
    rope = rope_cache(luc, cfg.head_dim)
    cos, sin = rope.cos.cpu().numpy(), rope.sin.cpu().numpy()
    qkv, kp, vp = h.qkv.copy(), h.k_pool.copy(), h.v_pool.copy()
    out = orc.decode_step(qkv, None, None, None, cos, sin, kp, vp, h.tables, h.positions, layer,
                          cfg.hq, cfg.hkv, cfg.head_dim, sm_scale(cfg.head_dim), 16, h.num_layers,
                          cfg.dtype)
    return dict(out=out, qkv=qkv, k_pool=kp, v_pool=vp)


def max_abs(orc, a_bits, b_bits, dtype):
    a = orc.to_f32(a_bits, dtype).astype(np.float64)
    b = orc.to_f32(b_bits, dtype).astype(np.float64)
    return float(np.max(np.abs(a - b)))


def storage_ulp(x, dtype):
    """The spacing of the storage type (bf16: 8 significant bits, fp16: 11,
    normal range) at magnitude |x|, for float64 arrays."""
    mant = 8 if dtype == "bf16" else 11
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    if dtype == "f16":
        e = np.maximum(e, -14)  # fp16 subnormals: fixed spacing 2^-24
    return 2.0 ** (e - (mant - 1))


def ulp_gate(orc, got_bits, want_bits, dtype, max_ulps=4, max_frac=None):
    """Attention outputs [rows, heads, d] against the oracle's, in storage
    units at the row's scale: |got - want| over the storage spacing at
    max(|want|, rms), rms being the root mean square of that (row, head)'s
    output vector.  Every element must be within `max_ulps` such units and,
    with max_frac, at most that fraction of the elements may differ at all.

    Why units at the row's scale: the MFMA paths round each softmax weight p
    to the storage type before the PV product (the 16-bit B operand), the
    reference keeps it in f32.  With a relative error up to 2^-9 (bf16) or
    2^-12 (fp16) per weight, the output moves by about 0.3 storage units at
    the row's RMS (standard deviation), independent of the context length,
    and an element near zero shows the same absolute error.  A dropped or
    doubled token moves every element of a row by (v_t - o) / n: at n = 2048
    and |v_t - o| ~ 0.5 that is ~5.6 units at the row's RMS, so a gate of a
    few units still sees it in some element of every affected row.  The
    units at rms / 4 are reported too.  Returns the report line; asserts."""
    a = orc.to_f32(got_bits, dtype).astype(np.float64)
    b = orc.to_f32(want_bits, dtype).astype(np.float64)
    rms = np.sqrt(np.mean(b * b, axis=-1, keepdims=True))
    err = np.abs(a - b)
    units = err / storage_ulp(np.maximum(np.abs(b), rms), dtype)
    units4 = err / storage_ulp(np.maximum(np.abs(b), rms / 4), dtype)
    diff = int(np.count_nonzero(a != b))
    hist = [int(np.count_nonzero(units <= 0.5)), int(np.count_nonzero((units > 0.5) & (units <= 1.5))),
            int(np.count_nonzero((units > 1.5) & (units <= 2.5))), int(np.count_nonzero(units > 2.5))]
    line = (f"storage units at the row's rms: max {units.max():.3f} (at rms/4: {units4.max():.3f}), "
            f"elements <=0.5 / ~1 / ~2 / >2.5 units: {hist}, {diff} of {a.size} differ "
            f"({diff / a.size:.2%})")
    say("  " + line)
    assert np.all(np.isfinite(a) == np.isfinite(b)), "finite / non-finite outputs differ"
    assert units.max() <= max_ulps + 1e-9, line
    if max_frac is not None:
        assert diff <= max_frac * a.size, line
    return line
