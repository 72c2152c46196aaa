"""Needle tests of the decode path (inputs: tests/needle.py): one dominant
key per (sequence, kv head) at page, tile and split boundaries and at the new
token, with NaN in every unused slot; each head's output must be V[t*] bit
for bit.  Fused (luc_decode_step) and unfused (luc_rope_append +
luc_paged_decode) paths, automatic and forced split sizes, both head dims.
The addressing and merge under test are the reference's
(src/kernels/attention.cu:80-87 token and page addressing, :140-174
partition merge) generalised to splits."""
import numpy as np
import pytest

from lucciola_rs_amd import workloads as wl
from gpu_util import gpu_step, rope_cache, say
from needle import CASES, needle_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "unfused"])
@pytest.mark.parametrize("head_dim,dtype,hq,hkv,splits", CASES, ids=["d64_f16", "d128_bf16"])
def test_needle_at_page_tile_and_split_boundaries(luc, head_dim, dtype, hq, hkv, splits, fused):
    rope = rope_cache(luc, head_dim)
    cos, sin = rope.cos.cpu().numpy(), rope.sin.cpu().numpy()
    cfg = wl.DecodeConfig(f"needle_d{head_dim}", 24, hq, hkv, head_dim, dtype, 2, 4200,
                          24 * 263 + 8, 0.5)
    for seed in (1, 2):
        h, needles, want = needle_inputs(cfg, seed, cos, sin)
        for split in splits:
            got = gpu_step(luc, h, split_tokens=split, fused=fused)["out"]
            bad = np.argwhere(np.any(got != want, axis=2))
            say(f"  {len(np.unique(needles))} needle positions, split {split}: "
                f"{len(bad)} of {cfg.batch * cfg.hq} heads differ")
            for b, q in bad[:4]:
                kv = q // (cfg.hq // cfg.hkv)
                say(f"    seq {b} ctx {h.ctx[b]} head {q}: needle at {needles[b, kv]}")
            assert len(bad) == 0
