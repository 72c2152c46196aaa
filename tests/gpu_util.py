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
