"""The generator and the oracle reproduce the committed golden fixtures (tests/golden/).

The fixtures are written by tests/golden/make_golden.py; a change in the
generator (layout digest) or in the oracle's numbers shows up here first.
"""

import dataclasses
import json
from pathlib import Path

import numpy as np
import pytest

import kbench_oracle as O
from kbench import synth

GOLDEN = Path(__file__).resolve().parent / "golden"
INDEX = json.loads((GOLDEN / "index.json").read_text())


@pytest.mark.parametrize("key", sorted(INDEX))
def test_generator_digest_and_summary(key):
    rec = INDEX[key]
    cfg = synth.config(rec["config"])
    if rec["statewise"] is not None:
        cfg = dataclasses.replace(cfg, statewise=rec["statewise"])
    p = synth.build_problem(cfg)
    assert synth.layout_digest(p) == rec["digest"]
    assert synth.summary(p) == rec["summary"]


@pytest.mark.parametrize("key", sorted(INDEX))
def test_oracle_reproduces_fixture(key):
    rec = INDEX[key]
    cfg = synth.config(rec["config"])
    if rec["statewise"] is not None:
        cfg = dataclasses.replace(cfg, statewise=rec["statewise"])
    p = synth.build_problem(cfg)
    prob = O.Problem.from_dict(p)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    ref = np.load(GOLDEN / f"{key}.npz")
    loss, saved = O.forward(prob, theta, cw)
    assert abs(loss - float(ref["loss"])) <= 1e-11 * abs(float(ref["loss"]))
    assert np.allclose(saved["E"], ref["E"], rtol=0, atol=1e-12)
    assert int(saved["n_e_iter"]) == int(ref["n_e_iter"])
    gt, gc, info = O.backward(prob, theta, cw, saved)
    assert np.allclose(gt, ref["grad_theta"], rtol=1e-10, atol=1e-12)
    assert np.allclose(gc, ref["grad_col"], rtol=1e-10, atol=1e-12)
    assert int(info["n_bicgstab"]) == int(ref["n_bicgstab"])
