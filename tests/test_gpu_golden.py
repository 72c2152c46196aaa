"""The single_512 known answer (tests/golden/single_512.json) through the C
ABI on the GPU: one luc_decode_step of the single-sequence workload (14q/2kv,
d=64, fp16, context 512 over 32 permuted pages).  The roped q and the new
cache slot must equal the recorded bits; the attention output must lie within
the fp16 tolerance (2e-3 max-abs) of the recorded output."""
import numpy as np
import pytest
import torch

import golden_single_512 as g
from gpu_util import say

pytestmark = pytest.mark.gpu


def test_decode_step_matches_the_known_answer(luc):
    from lucciola_rs_amd import workloads as wl
    from lucciola_rs_amd.engine import RopeCache, decode_step

    fx = g.fixture()
    cfg, h = g.inputs()
    dev = torch.device("cuda:0")
    t = lambda a: wl.bits_to_tensor(a, cfg.dtype).to(dev)  # noqa: E731
    qkv, kp, vp = t(h.qkv), t(h.k_pool), t(h.v_pool)
    tables = torch.from_numpy(h.tables).to(dev)
    pos = torch.from_numpy(h.positions).to(dev)
    out = torch.empty((1, cfg.hq * cfg.head_dim), dtype=cfg.torch_dtype, device=dev)
    rope = RopeCache(1024, cfg.head_dim, cfg.rope_theta, lib=luc, device=dev)
    max_ctx = int(h.ctx.max())
    say(f"  [gpu] single_512 known answer: decode_step, ctx {max_ctx}")
    for split in (0, 64):  # the automatic split and 64-token splits (8 splits)
        q_in, k_in, v_in = qkv.clone(), kp.clone(), vp.clone()
        ws = luc.workspace(1, cfg.hq, cfg.hkv, cfg.head_dim, max_ctx, split_tokens=split)
        decode_step(q_in, None, None, None, rope, k_in, v_in, tables, pos, max_ctx, 0, 1, cfg.hq,
                    cfg.hkv, cfg.head_dim, out, ws, split_tokens=split, lib=luc)
        torch.cuda.synchronize()
        bits = lambda x: x.cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
        p = int(h.positions[0])
        page = int(h.tables[0, p // 16])
        assert np.array_equal(bits(q_in)[0, : cfg.hq * cfg.head_dim], np.array(fx["q_roped_bits"], np.uint16))
        assert np.array_equal(bits(k_in)[page, 0, :, p % 16].reshape(-1), np.array(fx["k_slot_bits"], np.uint16))
        assert np.array_equal(bits(v_in)[page, 0, :, p % 16].reshape(-1), np.array(fx["v_slot_bits"], np.uint16))
        want = wl.bits_to_tensor(np.array(fx["out_bits"], np.uint16), cfg.dtype).float().numpy()
        err = float(np.max(np.abs(out.float().cpu().numpy().reshape(-1) - want)))
        say(f"    split {split}: max |out - known answer| {err:.2e}")
        assert err <= 2e-3
