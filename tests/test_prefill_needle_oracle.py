"""CPU pins of the prefill needle inputs (tests/prefill_needle.py): the
oracle's prefill gives V[t*] bit for bit in every row at or past each needle
and something else in every row before it, and oracle mutants with a planted
causal-range, addressing or head-mapping mistake (ORC_MUTANT in
oracle/luc_oracle.c) fail them, so a needle catches the kind of mistake it is
placed to catch."""
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from lucciola_rs_amd import workloads as wl
from lucciola_rs_amd.engine import sm_scale
from prefill_needle import needle_mismatches, needle_prefill_inputs

SRC = os.path.join(os.path.dirname(oracle.__file__), "luc_oracle.c")
SHAPES = [(64, "bf16", 14, 2), (128, "f16", 12, 2)]


def mismatches(o, seeds=(1,)):
    """(late, early) needle mismatches of the oracle's prefill over both shapes."""
    late = early = 0
    for d, dt, hq, hkv in SHAPES:
        cos, sin = o.rope_table(1024, d, 1e6)
        cfg = wl.PrefillConfig(f"pneedle_d{d}", 8, 0, hq, hkv, d, dt, 0, 0, 0.5)
        for seed in seeds:
            h, needles, vsel = needle_prefill_inputs(cfg, seed, cos, sin)
            qkv, kp, vp = h.qkv.copy(), h.k_pool.copy(), h.v_pool.copy()
            out = o.prefill(qkv, None, None, None, cos, sin, kp, vp, h.tables, h.cu_seqlens,
                            h.start_pos, 0, hq, hkv, d, sm_scale(d), 16, 1, dt)
            a, b = needle_mismatches(h, needles, vsel, out.reshape(-1, hq, d))
            late, early = late + a, early + b
    return late, early


def test_oracle_reproduces_prefill_needles(orc):
    assert mismatches(orc, seeds=(1, 2)) == (0, 0)


_CHILD = """
import sys
sys.path[:0] = {paths!r}
import __graft_entry__
__graft_entry__.load_package()
import oracle
import test_prefill_needle_oracle as t
print("MISMATCHES", *t.mismatches(oracle.Oracle({so!r})))
"""

MUTANTS = {4: "slot offset: head and token strides swapped", 7: "last context token dropped",
           9: "wrong GQA head -> kv head mapping",
           17: "prefill rows attend one token past their own position"}


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_prefill_needles_catch_oracle_mutant(mutant, tmp_path):
    so = tmp_path / f"mutant{mutant}.so"
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-fopenmp", "-ffp-contract=off",
                    f"-DORC_MUTANT={mutant}", "-shared", "-o", str(so), SRC, "-lm"], check=True)
    here = os.path.dirname(os.path.abspath(__file__))
    code = _CHILD.format(paths=[here, os.path.dirname(here)], so=str(so))
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=600)
    if res.returncode < 0:
        return  # an out-of-bounds access crashed the child: caught
    assert res.returncode == 0, res.stderr[-3000:]
    late, early = map(int, [l for l in res.stdout.splitlines() if l.startswith("MISMATCHES")][-1].split()[1:])
    assert late + early > 0, f"mutant {mutant} ({MUTANTS[mutant]}) reproduces every prefill needle"
