"""Writes tests/golden/single_512.json, the known answer of one decode step of
the single-sequence workload: 14 q / 2 kv heads, head_dim 64, fp16, context
512 over a seeded permutation of 32 pages (page size 16), values N(0,1)*0.5,
RoPE theta 1e6, softmax scale 1/8.

The step is the reference's per-token path (src/models.rs:505-549): bias-free
RoPE of q and k at position 511 (src/kernels/rope.cu), the cache write of k
and v at that slot (src/kernels/kv_cache.cu), then attention over positions
0..511 (src/kernels/attention.cu).  The answer comes from the CPU oracle; the
script refuses to write it unless the oracle's output agrees with f64 textbook
attention on the same cache within 1e-3 (the RoPE and the slot write are
pinned by tests/pins.py).

The fixture holds the seed, SHA-256 digests of the regenerated inputs (so a
change of the input generator is caught rather than silently compared), and
the output bits: the attention output, the roped q row and the new k/v slot.

    python tests/golden/make_single_512.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

SEED = 512
OUT = os.path.join(HERE, "single_512.json")


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def inputs():
    import __graft_entry__
    __graft_entry__.load_package()
    from lucciola_rs_amd import workloads as wl
    cfg = wl.CONFIGS["single_512"]
    return cfg, wl.host_decode_inputs(cfg, SEED, poison=False)


def oracle_step(orc, cfg, h):
    """(output bits [hq*d], q row bits after RoPE [hq*d], k slot, v slot)."""
    from lucciola_rs_amd.engine import sm_scale
    cos, sin = orc.rope_table(cfg.ctx_hi + 1, cfg.head_dim, cfg.rope_theta)
    qkv, kp, vp = h.qkv.copy(), h.k_pool.copy(), h.v_pool.copy()
    out = orc.decode_step(qkv, None, None, None, cos, sin, kp, vp, h.tables, h.positions, 0,
                          cfg.hq, cfg.hkv, cfg.head_dim, sm_scale(cfg.head_dim), 16, 1, cfg.dtype)
    pos = int(h.positions[0])
    page = int(h.tables[0, pos // 16])
    return (out.reshape(-1), qkv[0, : cfg.hq * cfg.head_dim].copy(), kp[page, 0, :, pos % 16].copy(),
            vp[page, 0, :, pos % 16].copy(), kp, vp)


def main():
    import oracle
    import pins
    orc = oracle.get()
    cfg, h = inputs()
    out, q, kslot, vslot, kp, vp = oracle_step(orc, cfg, h)
    # f64 textbook attention over the cache after the step, with the roped q
    d, g = cfg.head_dim, cfg.hq // cfg.hkv
    qf = pins.f32(q, cfg.dtype).astype(np.float64).reshape(cfg.hq, d)
    worst = 0.0
    for qh in range(cfg.hq):
        k, v = pins.gather_kv(kp, vp, h.tables[0], 0, qh // g, int(h.ctx[0]), cfg.dtype)
        want = pins.textbook_attention(qf[qh], k, v, 1.0 / np.sqrt(d))
        got = pins.f32(out[qh * d:(qh + 1) * d], cfg.dtype)
        worst = max(worst, float(np.max(np.abs(got - want))))
    assert worst <= 1e-3, f"oracle vs f64 textbook attention: {worst}"
    assert kslot.shape == (cfg.hkv, d) and vslot.shape == (cfg.hkv, d)
    fixture = {
        "workload": cfg.name, "seed": SEED, "dtype": cfg.dtype,
        "shape": {"q_heads": cfg.hq, "kv_heads": cfg.hkv, "head_dim": d, "ctx": int(h.ctx[0]),
                  "page_size": 16, "pages": int(h.tables.shape[1])},
        "inputs_sha256": {"qkv": digest(h.qkv), "k_pool": digest(h.k_pool),
                          "v_pool": digest(h.v_pool), "tables": digest(h.tables)},
        "f64_textbook_max_abs": worst,
        "out_bits": [int(x) for x in out],
        "q_roped_bits": [int(x) for x in q],
        "k_slot_bits": [int(x) for x in kslot.reshape(-1)],
        "v_slot_bits": [int(x) for x in vslot.reshape(-1)],
    }
    with open(OUT, "w") as f:
        json.dump(fixture, f, separators=(",", ":"))
    print(f"wrote {OUT}: max |oracle - f64| = {worst:.2e}")


if __name__ == "__main__":
    main()
