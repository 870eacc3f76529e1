"""The oracle's GMRES self-loop solver (pristine wave_backward.py:574-653, 1136-1188) against what fixes it.

* ``gmres_fixed`` with as many iterations as unknowns solves a random
  nonsymmetric system exactly (dense solve), its residual never grows with
  the iteration count, and b = 0 or no iterations give 0;
* in the backward, GMRES solves (I - J^T) v = rhs: with enough iterations the
  solve's gradients equal those of a long Neumann series (both are the exact
  implicit gradient, also pinned against finite differences of the loss), and
  a short GMRES differs from the equally short Neumann truncation.
"""

import numpy as np
import pytest

import kbench_oracle as O
import kbtest


def _system(n, seed=0):
    g = np.random.default_rng(seed)
    A = np.eye(n) + 0.3 * g.normal(size=(n, n)) / np.sqrt(n)
    return A, g.normal(size=n)


def test_gmres_full_dimension_is_an_exact_solve():
    A, b = _system(30)
    x = O.gmres_fixed(lambda v: A @ v, b, 30)
    assert np.abs(x - np.linalg.solve(A, b)).max() <= 1e-10 * np.abs(b).max()
    # the solution keeps b's shape (a wave is a [W, S] block)
    X = O.gmres_fixed(lambda v: (A @ v.reshape(-1)).reshape(5, 6), b.reshape(5, 6), 30)
    assert X.shape == (5, 6) and np.abs(X.reshape(-1) - x).max() <= 1e-12


def test_gmres_residual_never_grows():
    A, b = _system(40, seed=1)
    res = [np.linalg.norm(b - A @ O.gmres_fixed(lambda v: A @ v, b, m)) for m in range(1, 16)]
    assert all(r2 <= r1 * (1 + 1e-12) for r1, r2 in zip(res, res[1:]))
    assert res[-1] < 1e-3 * res[0]


def test_gmres_zero_cases():
    A, b = _system(8)
    assert not O.gmres_fixed(lambda v: A @ v, np.zeros(8), 5).any()
    assert not O.gmres_fixed(lambda v: A @ v, b, 0).any()


def _backward(solver, terms, theta=None, cw=None):
    p = kbtest.problem("tiny")
    prob = O.Problem.from_dict(p)
    prob.so.update(pi_iters=120, neumann_terms=terms, use_adjoint_pruning=False, adjoint_pruning_threshold=0.0,
                   bicgstab_tol=1e-13, e_tol=1e-14, self_loop_solver=solver)
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float64) if theta is None else theta
    cw = np.linspace(-0.7, 0.9, prob.S) if cw is None else cw
    loss, saved = O.forward(prob, theta, cw)
    gt, gc, _ = O.backward(prob, theta, cw, saved)
    return prob, theta, cw, gt, gc


def test_converged_gmres_gradient_is_the_implicit_gradient():
    _, theta, cw, gt_n, gc_n = _backward("neumann", 200)
    prob, _, _, gt_g, gc_g = _backward("gmres", 40)
    assert np.abs(gt_g - gt_n).max() <= 1e-9 * np.abs(gt_n).max()
    assert np.abs(gc_g - gc_n).max() <= 1e-9 * np.abs(gc_n).max()
    # and against central differences of the converged loss
    h = 1e-5
    fd = np.zeros_like(theta)
    for idx in np.ndindex(theta.shape):
        tp, tm = theta.copy(), theta.copy()
        tp[idx] += h
        tm[idx] -= h
        fd[idx] = (O.forward(prob, tp, cw)[0] - O.forward(prob, tm, cw)[0]) / (2 * h)
    assert np.abs(gt_g - fd).max() <= 1e-6 * np.abs(fd).max()


def test_short_gmres_is_not_the_short_neumann_series():
    *_, gt_n, _ = _backward("neumann", 2)
    *_, gt_g, _ = _backward("gmres", 2)
    *_, gt_x, _ = _backward("neumann", 200)
    assert np.abs(gt_g - gt_n).max() > 1e-6 * np.abs(gt_n).max()
    # two Krylov steps already beat the two-term series against the exact gradient
    assert np.abs(gt_g - gt_x).max() < np.abs(gt_n - gt_x).max()


def test_unknown_solver_is_refused():
    with pytest.raises(ValueError):
        _backward("cg", 3)
