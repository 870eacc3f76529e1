"""``synth.level_waves``: one wave per clade-DAG level gives every row the same result as the size waves.

A row of the truncated forward and of its adjoint depends only on its own
children, which sit on lower levels, so regrouping the rows changes the
number of waves (and of wrapper calls) but no row's arithmetic: the oracle's
loss and every Pi / Pibar row are bitwise equal and the gradients equal up to
the order of the cross-wave sums.
"""

import numpy as np
import pytest

import kbench_oracle as O
from kbench import synth
import kbtest


@pytest.mark.parametrize("name,statewise", [("tiny", None), ("1", None), ("1", True)])
def test_level_waves_solve_is_the_size_waves_solve(name, statewise):
    p = kbtest.problem(name, statewise)
    q, new_of_old = synth.level_waves(p)
    wp, wq = p["static"]["wave_layout"], q["static"]["wave_layout"]
    assert len(wq["wave_metas"]) <= len(wp["wave_metas"])
    assert sorted(new_of_old.tolist()) == list(range(new_of_old.size))
    A, B = O.Problem.from_dict(p), O.Problem.from_dict(q)
    th = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw = np.linspace(-0.5, 0.5, A.S)
    la, sa = O.forward(A, th, cw)
    lb, sb = O.forward(B, th, cw)
    assert la == lb
    for k in ("pi_wave", "pibar_wave", "pibar_row_max"):
        assert np.array_equal(sa[k], sb[k][new_of_old], equal_nan=True), k
    ga, gca, _ = O.backward(A, th, cw, sa)
    gb, gcb, _ = O.backward(B, th, cw, sb)
    assert np.abs(ga - gb).max() <= 1e-12 * np.abs(ga).max()
    assert np.abs(gca - gcb).max() <= 1e-12 * np.abs(gca).max()


def test_level_waves_are_dependency_levels():
    p = kbtest.problem("1")
    q, _ = synth.level_waves(p)
    wl = q["static"]["wave_layout"]
    wave_of = np.empty(int(np.asarray(wl["item_idx"]).shape[0]), dtype=np.int64)
    for i, m in enumerate(wl["wave_metas"]):
        wave_of[int(m["start"]):int(m["start"]) + int(m["W"])] = i
    for i, m in enumerate(wl["wave_metas"]):
        if "sl" not in m:
            assert i == 0  # only the leaf rows have no splits
            continue
        children = np.concatenate([np.asarray(m["sl"]), np.asarray(m["sr"])])
        assert (wave_of[children] < i).all()  # children on lower levels
        # some row of every wave above the leaves has a child on the level just below
        assert (wave_of[children] == i - 1).any()
    # one wave per level: the levels are 0..depth, the wave count the DAG depth + 1
    assert synth.summary(q)["n_waves"] == len(wl["wave_metas"])


def test_level_waves_keep_the_root_rows_and_chunk_on_request():
    p = kbtest.problem("1")
    q, new_of_old = synth.level_waves(p, max_wave_rows=64)
    roots_p = np.asarray(p["static"]["wave_layout"]["root_row_ids"])
    roots_q = np.asarray(q["static"]["wave_layout"]["root_row_ids"])
    assert np.array_equal(roots_q, new_of_old[roots_p])
    assert max(int(m["W"]) for m in q["static"]["wave_layout"]["wave_metas"]) <= 64
