"""The oracle reproduces the reference's own forward on configs 1 and 2 (tests/golden/pristine_fwd_*.npz).

The fixtures hold the outputs of the reference's frozen glue over its pristine
Triton kernels (kbench/runtime.py:63-75, experiments/pristine_kernels/*.py),
run in float32 under the Triton interpreter by
tests/golden/make_pristine_fwd.py on problems this repository generates.
They pin what no closed form fixes: the truncated forward schedule
(``pi_iters - 1`` sweeps per wave, leaf waves from the leaf initialisation,
split waves from their split term, forward.py:60-117), at two sweep counts
whose losses differ by 1.4e-3 relative, so a wrong sweep count, a dropped
split term or a wrong starting row fails here.  Config 2 (S = 511, rows with
several splits, E stopping tolerance 1e-6) adds the split reduction over
several splits and a second E tolerance; its fixture keeps every row maximum,
the root rows of Pi and Pibar and 192 seeded other rows (``rows``).

Tolerances follow from the reference's float32 arithmetic: loss relative
1e-6, arrays |a - b| <= 1e-5 max(1, |b|), and the same non-finite pattern
(the E_s1 / E_s2 rows of the leaves are -inf in both).
"""

import dataclasses
from pathlib import Path

import numpy as np
import pytest

import kbench_oracle as O
from kbench import synth

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = {"config1": ("1", None), "config1_pi4": ("1", None), "config1_statewise": ("1", True),
         "config2": ("2", None)}
ARRAYS = ("E", "E_s1", "E_s2", "Ebar", "pi_wave", "pibar_wave", "pibar_row_max")


def fixture(case: str):
    return np.load(GOLDEN / f"pristine_fwd_{case}.npz")


def problem(case: str) -> dict:
    name, statewise = CASES[case]
    cfg = synth.config(name)
    if statewise is not None:
        cfg = dataclasses.replace(cfg, statewise=statewise)
    return synth.build_problem(cfg)


def rows_of(z, k, got):
    """``got`` restricted to the rows the fixture keeps for array ``k`` (all rows unless it has ``rows``)."""
    got = np.asarray(got)
    if "rows" in z.files and k in ("pi_wave", "pibar_wave"):
        return got[np.asarray(z["rows"])]
    return got


def close_to_fixture(got, ref, rel=1e-5):
    """(same non-finite pattern, max |got - ref| / max(1, |ref|) over the finite entries)."""
    got = np.asarray(got, dtype=np.float64).reshape(ref.shape)
    ref = np.asarray(ref, dtype=np.float64)
    fin = np.isfinite(ref)
    pattern = bool((np.isfinite(got) == fin).all() and (got[~fin] == ref[~fin]).all())
    err = float((np.abs(got[fin] - ref[fin]) / np.maximum(1.0, np.abs(ref[fin]))).max()) if fin.any() else 0.0
    return pattern, err


@pytest.mark.parametrize("case", sorted(CASES))
def test_oracle_reproduces_the_reference_forward(case):
    z = fixture(case)
    p = problem(case)
    assert synth.layout_digest(p) == str(z["digest"])
    prob = O.Problem.from_dict(p)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    loss, saved = O.forward(prob, z["theta"].astype(np.float64), cw, pi_iters=int(z["pi_iters"]))
    assert abs(loss - float(z["loss"])) <= 1e-6 * abs(float(z["loss"]))
    for k in ARRAYS:
        pattern, err = close_to_fixture(rows_of(z, k, saved[k]), z[k])
        assert pattern and err <= 1e-5, (k, pattern, err)


def test_sweep_count_is_visible_in_the_fixtures():
    """The pi_iters 4 and 16 fixtures differ well beyond the tolerance, and the oracle tells them apart."""
    a, b = fixture("config1"), fixture("config1_pi4")
    assert abs(float(a["loss"]) - float(b["loss"])) >= 1e-3 * abs(float(a["loss"]))
    prob = O.Problem.from_dict(problem("config1"))
    cw = np.asarray(problem("config1")["inputs"]["col_weights"], dtype=np.float64)
    loss6, _ = O.forward(prob, a["theta"].astype(np.float64), cw, pi_iters=6)
    assert abs(loss6 - float(a["loss"])) > 1e-5 * abs(float(a["loss"]))
    assert abs(loss6 - float(b["loss"])) > 1e-5 * abs(float(b["loss"]))
