"""Pins of the oracle's ``pibar_side_threshold`` rule (CPU).

The glue's option (reference kbench/api/_implicit_grad.py:300-353) drops a split
side from the Pibar VJP when the abs-sum of its staged u_d over the states is
not above the threshold (pristine wave_backward.py:1777-1779, 1877-1884, and
the early return at 2263-2266).  These checks fix the oracle's reading of it:

* a threshold below every nonzero side bound gives bitwise the threshold-0
  gradient (the sides it drops have all-zero u_d and contribute nothing);
* a threshold above every side bound drops every side: the gradient then
  equals the threshold-0 backward with every Pibar VJP row subtracted again
  from the children's adjoint rows and the column gradient (so a rule that
  dropped the wrong term, or kept a side, fails);
* between the two, the number of sides kept falls as the threshold rises and
  the gradient changes.
"""

import dataclasses

import numpy as np

import kbtest


def _backward(name, thr, statewise=True):
    import kbench_oracle as O

    p = kbtest.problem(name, statewise)
    prob, _, saved = kbtest.oracle_forward(name, statewise)
    prob = dataclasses.replace(prob, so=dict(prob.so, pibar_side_threshold=float(thr)))
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    gt, gc, _info, extra = O.backward(prob, theta, cw, saved, collect=True)
    return gt, gc, extra


def _bounds(extra):
    return np.concatenate(extra["side_bounds"]) if extra["side_bounds"] else np.zeros(0)


def test_tiny_threshold_is_the_zero_threshold():
    gt0, gc0, ex0 = _backward("1", 0.0)
    b = _bounds(ex0)
    nz = b[b > 0]
    assert nz.size > 0
    gt, gc, _ = _backward("1", float(nz.min()) * 0.5)
    assert np.array_equal(gt, gt0) and np.array_equal(gc, gc0)


def test_huge_threshold_drops_every_pibar_vjp_row(monkeypatch):
    import kbench_oracle as O

    gt0, gc0, ex0 = _backward("1", 0.0)
    gt_all_off, gc_all_off, _ = _backward("1", float(_bounds(ex0).max()) * 2.0 + 1.0)
    # independent reading: the threshold-0 backward with every Pibar VJP row taken back out of
    # the children's adjoint rows and the column gradient
    real_cross = O.dts_cross_backward

    def cross_without_tree(*a, **k):
        out = real_cross(*a, **k)
        for side, key in (("l", "rhs_l"), ("r", "rhs_r")):
            out[key] = out[key] - out["tree_" + side]
            out["col_grad"] = out["col_grad"] - out["tree_" + side].sum(axis=0)
        return out

    monkeypatch.setattr(O, "dts_cross_backward", cross_without_tree)
    gt_ref, gc_ref, _ = _backward("1", 0.0)
    monkeypatch.setattr(O, "dts_cross_backward", real_cross)
    assert np.allclose(gt_all_off, gt_ref, rtol=1e-12, atol=1e-12 * np.abs(gt_ref).max())
    assert np.allclose(gc_all_off, gc_ref, rtol=1e-12, atol=1e-12 * np.abs(gc_ref).max())
    assert kbtest.norm_rel(gt_all_off, gt0) > 1e-6  # the tree term matters on this problem


def test_sides_kept_fall_as_the_threshold_rises():
    _, _, ex0 = _backward("1", 0.0)
    b = _bounds(ex0)
    qs = np.quantile(b[b > 0], [0.25, 0.5, 0.75])
    kept = [int((b > q).sum()) for q in qs]
    assert kept[0] > kept[1] > kept[2] > 0
    g_prev = None
    for q in qs:
        gt, _, ex = _backward("1", float(q))
        assert np.array_equal(_bounds(ex) > 0, b > 0)  # the bounds come from the same staged u_d
        if g_prev is not None:
            assert not np.array_equal(gt, g_prev)
        g_prev = gt
