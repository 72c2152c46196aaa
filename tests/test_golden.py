"""Known answer of the single-sequence decode step (tests/golden/single_512.json,
written by tests/golden/make_single_512.py): the regenerated inputs must hash
to the recorded digests, and the oracle must reproduce the recorded output,
roped q and cache slot bit for bit."""
import json
import os

import numpy as np

import golden_single_512 as g


def test_inputs_regenerate_to_the_recorded_digests():
    fx = g.fixture()
    _, h = g.inputs()
    for name, arr in (("qkv", h.qkv), ("k_pool", h.k_pool), ("v_pool", h.v_pool),
                      ("tables", h.tables)):
        assert g.digest(arr) == fx["inputs_sha256"][name], name


def test_oracle_reproduces_the_known_answer(orc):
    fx = g.fixture()
    cfg, h = g.inputs()
    out, q, kslot, vslot, _, _ = g.oracle_step(orc, cfg, h)
    assert np.array_equal(out, np.array(fx["out_bits"], np.uint16))
    assert np.array_equal(q, np.array(fx["q_roped_bits"], np.uint16))
    assert np.array_equal(kslot.reshape(-1), np.array(fx["k_slot_bits"], np.uint16))
    assert np.array_equal(vslot.reshape(-1), np.array(fx["v_slot_bits"], np.uint16))
    assert fx["f64_textbook_max_abs"] <= 1e-3
