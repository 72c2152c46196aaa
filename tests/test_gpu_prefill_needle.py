"""Needle tests of the prefill path (inputs: tests/prefill_needle.py): one
dominant key per (sequence, kv head) at page, 32-row tile, 64-token block
and super-block edges, at the first prompt row and the last cached token,
and on the diagonal (a row's own position), after ragged cached prefixes,
with NaN in every unused slot.  Every row whose causal context holds the
needle must output V[t*] bit for bit in every q-head of the unit; every row
before it must not.  Both head dims and dtypes, several seeds.  Semantics:
the reference's per-token loop (src/models.rs:485-550) and its causal
addressing (src/kernels/attention.cu:80-87)."""
import numpy as np
import pytest
import torch

from lucciola_rs_amd import workloads as wl
from gpu_util import rope_cache, say
from prefill_needle import needle_mismatches, needle_prefill_inputs
from test_gpu_prefill import gpu_prefill

pytestmark = pytest.mark.gpu

SHAPES = [(64, "bf16", 14, 2), (64, "f16", 14, 2), (128, "bf16", 12, 2), (128, "f16", 28, 4)]


@pytest.fixture(autouse=True)
def _needs_device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


@pytest.mark.parametrize("head_dim,dtype,hq,hkv", SHAPES,
                         ids=[f"d{d}_{dt}_{a}q{b}kv" for d, dt, a, b in SHAPES])
def test_prefill_needle_at_page_tile_block_and_diagonal(luc, head_dim, dtype, hq, hkv):
    rope = rope_cache(luc, head_dim)
    cos, sin = rope.cos.cpu().numpy(), rope.sin.cpu().numpy()
    cfg = wl.PrefillConfig(f"pneedle_d{head_dim}", 8, 0, hq, hkv, head_dim, dtype, 0, 0, 0.5)
    placed = set()
    for seed in (1, 2, 3, 4):
        h, needles, vsel = needle_prefill_inputs(cfg, seed, cos, sin)
        got = gpu_prefill(luc, h)
        late, early = needle_mismatches(h, needles, vsel, got["out"])
        placed |= {(int(s), int(t)) for s, t in zip(np.repeat(h.start_pos, hkv), needles.reshape(-1))}
        say(f"  seed {seed}: needles {needles.tolist()}: {late} (row, head) pairs past a needle "
            f"differ from V[t*], {early} before it equal it")
        assert late == 0 and early == 0
    say(f"  {len(placed)} distinct (prefix, needle) placements")
