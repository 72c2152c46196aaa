"""Each planted oracle mistake (ORC_MUTANT=n in oracle/luc_oracle.c) must be
rejected by at least one of the pinning checks in tests/pins.py.  This shows
the checks pin the oracle rather than restate it."""
import os
import subprocess
import sys

import pytest

import oracle
import pins

SRC = os.path.join(os.path.dirname(oracle.__file__), "luc_oracle.c")

MUTANTS = {
    1: "score not scaled by sm_scale",
    2: "bias added after the rotation",
    3: "rotation sign flipped",
    4: "slot offset: head and token strides swapped",
    5: "partition merge without exp rescale",
    6: "V bias dropped in the cache write",
    7: "last context token dropped",
    8: "scores read from the V pool",
    9: "wrong GQA head -> kv head mapping",
    10: "fp16 rounding truncates",
    11: "RMSNorm mean over n - 1",
    12: "silu with exp(+x)",
    13: "argmax ties go to the higher thread",
    14: "top-k filter: ties go to the higher lane in the warp trees",
    15: "bitonic network: block directions swapped",
    16: "top-p cutoff needs cdf strictly above top_p",
    17: "prefill rows attend one token past their own position",
}


def all_checks(o):
    """(name, passed) for every pinning check, on small inputs."""
    res = []
    res.append(("rope_table", pins.check_rope_table(o, max_pos=256) <= 1))
    for dt in ("f16", "bf16"):
        res.append((f"rope_{dt}", pins.check_rope(o, dt) <= 1))
        res.append((f"kv_{dt}", pins.check_kv_update(o, dt) == 0))
        res.append((f"attn_{dt}", pins.check_attention(o, dt, 100) <= 1))
        res.append((f"sdpa_{dt}", pins.check_attention_sdpa(o, dt, 70) <= 1))
        res.append((f"inv_{dt}", pins.check_attention_invariants(o, dt) == 0))
        res.append((f"prefill_{dt}", pins.check_prefill(o, dt) <= 1))
    import numpy as np
    x = np.linspace(-3, 3, 10001, dtype=np.float32)
    res.append(("conv_f16", np.array_equal(o.to_storage(x, "f16"), pins.bits(x, "f16"))))
    res.append(("rmsnorm", pins.check_rmsnorm(o) <= 1))
    res.append(("silu_mul", pins.check_silu_mul(o) <= 1))
    res.append(("argmax", pins.check_argmax(o) == 0))
    res.append(("topk_filter", pins.check_topk_filter(o) == 0))
    res.append(("bitonic", pins.check_bitonic(o) == 0))
    res.append(("top_p", pins.check_top_p(o) == 0))
    return res


def test_unmutated_oracle_passes_all(orc):
    failed = [n for n, ok in all_checks(orc) if not ok]
    assert not failed, failed


# The checks of one mutant run in a child process: a planted indexing mistake
# can write outside the oracle's buffers and crash the process that runs it,
# which counts as caught (the unmutated oracle runs in-process above).
_CHILD = """
import sys
sys.path[:0] = {paths!r}
import oracle
import test_oracle_mutants as t
failed = [n for n, ok in t.all_checks(oracle.Oracle({so!r})) if not ok]
print("FAILED_CHECKS", ",".join(failed))
"""


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_mutant_is_caught(mutant, tmp_path):
    so = tmp_path / f"mutant{mutant}.so"
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-fopenmp", "-ffp-contract=off",
                    f"-DORC_MUTANT={mutant}", "-shared", "-o", str(so), SRC, "-lm"], check=True)
    here = os.path.dirname(os.path.abspath(__file__))
    code = _CHILD.format(paths=[here, os.path.dirname(here)], so=str(so))
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=600)
    if res.returncode < 0:
        return  # killed by a signal (an out-of-bounds write crashed the checks): caught
    assert res.returncode == 0, res.stderr[-3000:]
    line = [l for l in res.stdout.splitlines() if l.startswith("FAILED_CHECKS")][-1]
    failed = [n for n in line.split(" ", 1)[1].split(",") if n]
    assert failed, f"mutant {mutant} ({MUTANTS[mutant]}) passed every check"
