"""The backward's early stop of the Neumann series, restated on the float64 oracle.

The whole-pass backward (``kbench.fused.FusedSolver``, ``neumann_rtol``)
stops a row's series v = sum_n (J^T)^n rhs at the first term whose every
entry is at most rtol * max|rhs| of that row, the term included; the
reference sums all ``neumann_terms`` terms (pristine
wave_backward.py:1232-1269, the oracle's ``wave_backward_uniform``).  Here the
oracle's own backward runs with that rule in place of its loop, in float64,
so the effect of the rule alone is measured:

* with rtol = 0 the rule is the full series (bitwise the oracle's gradients);
* at the default rtol (2^-24) the gradients move by at most 3e-7 normwise,
  while rows stop after about half of their terms;
* a tolerance 2^14 times larger moves them measurably more (the check can
  tell the two apart).
"""

import numpy as np
import pytest

import kbench_oracle as O
import kbtest


def _rule(rtol, used):
    """``wave_backward_uniform`` with the kernel's stopping rule (same outputs)."""

    def wave_backward_uniform(Pi_s, Pibar_s, row_max, rhs, items, consts, tree, neumann_terms, *, active,
                              leaf_state=None, dts_r=None, solver="neumann"):
        assert solver == "neumann"
        co = O.self_loop_coeffs(Pi_s, Pibar_s, row_max, items, consts, tree, leaf_state=leaf_state, dts_r=dts_r)
        act = np.asarray(active, dtype=bool)[:, None]
        v = np.where(act, rhs, 0.0)
        tau = rtol * np.abs(v).max(axis=1, keepdims=True)
        term = v.copy()
        live = act.copy()
        n_used = np.zeros(v.shape[0], dtype=np.int64)
        for _ in range(int(neumann_terms)):
            if rtol > 0.0:
                live &= ~(np.abs(term) <= tau).all(axis=1, keepdims=True)
            if not live.any():
                break
            term = np.where(live, O.apply_JT(term, co, tree), 0.0)
            v = v + term
            n_used += live[:, 0]
        used.append(n_used[np.asarray(active, dtype=bool)])
        u = v * co.pcoef
        A = u.sum(axis=1, keepdims=True)
        col_grad = np.where(act, co.p_prime * (A - tree.subtree_sum(u)), 0.0).sum(axis=0)
        alpha = v * co.w_L
        aw = [np.where(act, alpha * ek * co.inv_sum, 0.0) for ek in co.e]
        return v, aw[0], aw[1], aw[2], aw[3] + aw[4] + aw[5], aw[3], aw[4], col_grad

    return wave_backward_uniform


def _problem(name):
    from kbench import synth

    if name == "config3_subset":
        return synth.family_subset(kbtest.problem("3", True), [0, 125, 250, 375])
    return kbtest.problem(name, True)


@pytest.mark.parametrize("name", ["1", "config3_subset"])
def test_early_stop_rule_on_the_oracle(name, monkeypatch):
    p = _problem(name)
    prob = O.Problem.from_dict(p)
    th = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    _, saved = O.forward(prob, th, cw)
    ref_t, ref_c, _ = O.backward(prob, th, cw, saved)
    n_terms = int(prob.so["neumann_terms"])
    out = {}
    for rtol in (0.0, 2.0 ** -24, 2.0 ** -10):
        used = []
        monkeypatch.setattr(O, "wave_backward_uniform", _rule(rtol, used))
        gt, gc, _ = O.backward(prob, th, cw, saved)
        u = np.concatenate(used)
        out[rtol] = (kbtest.norm_rel(gt, ref_t), kbtest.norm_rel(gc, ref_c), float(u.mean()), int(u.max()))
        print(f"  {name} rtol={rtol:.3g}: grad_theta rel={out[rtol][0]:.2e} grad_col rel={out[rtol][1]:.2e} "
              f"terms mean {out[rtol][2]:.2f} max {out[rtol][3]} of {n_terms}")
    assert out[0.0][:2] == (0.0, 0.0) and out[0.0][2] == n_terms
    d = 2.0 ** -24
    assert out[d][0] <= 3e-7 and out[d][1] <= 3e-7
    assert out[d][2] <= 0.7 * n_terms
    assert max(out[2.0 ** -10][:2]) > 10 * max(out[d][:2])
