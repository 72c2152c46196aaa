"""Needle inputs for the decode path: every key of a (sequence, kv head) is
zero except one token t*, whose key lies along the unit's query as the
kernels see it (q = 16 on four dims, roped at the new token's position; the
needle's key is that roped vector, or, when t* is the new token itself, its
k is q and both are roped together).  The score of t* is 1024 * sm_scale
(128 at head_dim 64, 90.5 at 128), every other score 0, so any other token
weighs less than e^-90 and the attention output of every q-head of the unit
is V[t*] itself, bit for bit.  t* is placed at the first and last token of
pages, tiles and splits of every size and at the new token; unused slots and
table entries hold NaN.  Shared by the GPU needle test and its CPU pin
against the oracle."""
import numpy as np

from lucciola_rs_amd import workloads as wl

PAGE = 16


def boundary_positions(ctx: int):
    """First and last tokens of pages, tiles and splits of every size that
    fall inside a context of ctx tokens, plus the first and newest tokens."""
    cand = {0, 1, ctx - 2, ctx - 1}
    for unit in (16, 32, 64, 128, 256, 512, 1024, 2048):
        for k in range(1, ctx // unit + 1):
            cand |= {k * unit - 1, k * unit}
    return sorted(p for p in cand if 0 <= p < ctx)


def needle_inputs(cfg, seed, cos, sin):
    """Host inputs whose keys are zero except one needle per (sequence, kv
    head); returns them, the needle of every unit and the expected output."""
    h = wl.host_decode_inputs(cfg, seed=seed, poison=True)
    d, G = cfg.head_dim, cfg.hq // cfg.hkv
    k_pool = h.k_pool.copy()
    k_pool[~np.isnan(wl.bits_to_tensor(k_pool, cfg.dtype).float().numpy())] = 0
    qkv = h.qkv.copy()
    qv = np.zeros(d, np.float64)
    qv[:4] = 16.0
    q_bits = wl.to_bits(qv.astype(np.float32), cfg.dtype)
    qkv[:, : cfg.hq * d] = np.tile(q_bits, cfg.hq)
    qkv[:, cfg.hq * d:(cfg.hq + cfg.hkv) * d] = 0  # the new token's k: zero
    needles = np.zeros((cfg.batch, cfg.hkv), np.int64)
    want = np.zeros((cfg.batch, cfg.hq, d), np.uint16)
    half = d // 2
    unit = 0
    for b in range(cfg.batch):
        pos = int(h.positions[b])
        cands = boundary_positions(pos + 1)
        for kv in range(cfg.hkv):
            t = pos if unit % 6 == 5 else cands[(unit * 7) % len(cands)]
            unit += 1
            needles[b, kv] = t
            v_row = slice((cfg.hq + cfg.hkv + kv) * d, (cfg.hq + cfg.hkv + kv + 1) * d)
            if t == pos:  # the new token: k = q, roped together at pos
                qkv[b, (cfg.hq + kv) * d:(cfg.hq + kv + 1) * d] = q_bits
                v = qkv[b, v_row]
            else:  # a cached key along q roped at pos (pairs i, i + d/2)
                c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
                key = np.concatenate([qv[:half] * c - qv[half:] * s, qv[:half] * s + qv[half:] * c])
                slot = (h.tables[b, t // PAGE], 0, kv, t % PAGE)
                k_pool[slot] = wl.to_bits(key.astype(np.float32), cfg.dtype)
                v = h.v_pool[slot]
            want[b, kv * G:(kv + 1) * G] = v
    return wl.HostDecode(cfg, 1, h.ctx, h.positions, h.tables, qkv, k_pool, h.v_pool), needles, want


CASES = [
    # (head_dim, dtype, q heads, kv heads, split sizes; 0 = the automatic choice)
    (64, "f16", 14, 2, (0, 256, 512, 1024, 2048)),
    (128, "bf16", 12, 2, (0, 128, 256, 512, 1024, 2048)),
]
