"""CPU pins of the needle inputs (tests/needle.py): the oracle reproduces
every expected output bit for bit, and oracle mutants with a planted
addressing or merge mistake (ORC_MUTANT in oracle/luc_oracle.c) fail them,
so a needle catches the kind of mistake it is placed to catch."""
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from lucciola_rs_amd import workloads as wl
from lucciola_rs_amd.engine import sm_scale
from needle import CASES, needle_inputs

SRC = os.path.join(os.path.dirname(oracle.__file__), "luc_oracle.c")


def mismatches(o, seeds=(1,)):
    """Heads whose oracle output differs from the needle's V, over both cases."""
    bad = 0
    for d, dt, hq, hkv, _ in CASES:
        cos, sin = o.rope_table(4300, d, 1e6)
        cfg = wl.DecodeConfig(f"needle_d{d}", 24, hq, hkv, d, dt, 2, 4200, 24 * 263 + 8, 0.5)
        for seed in seeds:
            h, _, want = needle_inputs(cfg, seed, cos, sin)
            qkv, kp, vp = h.qkv.copy(), h.k_pool.copy(), h.v_pool.copy()
            out = o.decode_step(qkv, None, None, None, cos, sin, kp, vp, h.tables, h.positions, 0,
                                hq, hkv, d, sm_scale(d), 16, 1, dt, 8)
            bad += int(np.sum(np.any(out != want, axis=2)))
    return bad


def test_oracle_reproduces_needles(orc):
    assert mismatches(orc, seeds=(1, 2)) == 0


_CHILD = """
import sys
sys.path[:0] = {paths!r}
import __graft_entry__
__graft_entry__.load_package()
import oracle
import test_needle_oracle as t
print("MISMATCHES", t.mismatches(oracle.Oracle({so!r})))
"""

MUTANTS = {4: "slot offset: head and token strides swapped", 5: "partition merge without exp rescale",
           7: "last context token dropped", 9: "wrong GQA head -> kv head mapping"}


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_needles_catch_oracle_mutant(mutant, tmp_path):
    so = tmp_path / f"mutant{mutant}.so"
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-fopenmp", "-ffp-contract=off",
                    f"-DORC_MUTANT={mutant}", "-shared", "-o", str(so), SRC, "-lm"], check=True)
    here = os.path.dirname(os.path.abspath(__file__))
    code = _CHILD.format(paths=[here, os.path.dirname(here)], so=str(so))
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=600)
    if res.returncode < 0:
        return  # an out-of-bounds write crashed the child: caught
    assert res.returncode == 0, res.stderr[-3000:]
    n = int([l for l in res.stdout.splitlines() if l.startswith("MISMATCHES")][-1].split()[1])
    assert n > 0, f"mutant {mutant} ({MUTANTS[mutant]}) reproduces every needle"
