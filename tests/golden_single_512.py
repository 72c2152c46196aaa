"""Shared helpers of the single_512 known-answer tests: the fixture, the
regenerated inputs and the oracle step (from tests/golden/make_single_512.py)."""
import importlib.util
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))
_spec = importlib.util.spec_from_file_location(
    "make_single_512", os.path.join(HERE, "golden", "make_single_512.py"))
_mk = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(_mk)

inputs = _mk.inputs
oracle_step = _mk.oracle_step
digest = _mk.digest


def fixture():
    with open(_mk.OUT) as f:
        return json.load(f)
