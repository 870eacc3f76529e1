"""Krylov solvers and Newton drivers on the CPU, against matrices and functions with known answers.

As the reference tests its CG witness on a 60x60 matrix of known spectrum
(its newton/test_witness.py:1-74), the solvers here run on Q diag(lam) Q^T
with chosen eigenvalues: solutions against a dense solve, the negative-
curvature certificate against the smallest eigenvalue, trust-region steps
against their radius, Lanczos extremes against the spectrum.  The drivers run
on smooth test functions with a known minimiser (objects with ``value`` /
``value_and_grad`` / ``hvp``, the ``Objective`` interface).
"""

import math

import numpy as np
import pytest
import torch

from kbench.newton import (cg_solve, cg_witness, lanczos_extremes, lanczos_min_eigpair, newton_cg, newton_lanczos,
                           newton_tr, steihaug_cg)


def _spectral(lams, seed=0):
    g = np.random.default_rng(seed)
    Q, _ = np.linalg.qr(g.normal(size=(len(lams), len(lams))))
    A = (Q * np.asarray(lams, dtype=np.float64)) @ Q.T
    return torch.as_tensor((A + A.T) / 2), torch.as_tensor(Q)


def _rhs(n, seed=1):
    return torch.as_tensor(np.random.default_rng(seed).normal(size=n))


def test_cg_solves_an_spd_system():
    A, _ = _spectral(np.linspace(0.5, 20.0, 60))
    b = _rhs(60)
    x, iters, ok = cg_solve(lambda v: A @ v, b, tol=1e-10, max_iter=200)
    ref = torch.linalg.solve(A, b)
    assert ok and iters <= 60 + 5
    assert float((x - ref).abs().max()) <= 1e-8 * float(ref.abs().max())
    x0 = ref + 1e-3 * _rhs(60, 2)
    x2, it2, ok2 = cg_solve(lambda v: A @ v, b, tol=1e-10, max_iter=200, x0=x0)
    assert ok2 and float((x2 - ref).abs().max()) <= 1e-8 * float(ref.abs().max())


def test_cg_witness_certifies_negative_curvature():
    lam_min, damp = -0.5, 0.1
    H, _ = _spectral(np.concatenate([[lam_min], np.linspace(0.2, 10.0, 59)]))
    A = H + damp * torch.eye(60, dtype=torch.float64)
    x, iters, status, cert = cg_witness(lambda v: A @ v, _rhs(60), tol=1e-10, max_iter=200)
    assert status == "neg_curv" and cert <= 0.0
    # d^T (H + damp) d / |d|^2 = cert  =>  lambda_min(H) <= cert - damp
    assert lam_min <= cert - damp + 1e-12
    # enough damping: positive definite, the witness solves like CG
    A2 = H + 0.6 * torch.eye(60, dtype=torch.float64)
    x2, _, status2, cert2 = cg_witness(lambda v: A2 @ v, _rhs(60), tol=1e-10, max_iter=200)
    assert status2 == "converged" and cert2 is None
    assert float((A2 @ x2 - _rhs(60)).abs().max()) <= 1e-8


def test_steihaug_statuses_and_products():
    b = _rhs(60)
    A, _ = _spectral(np.linspace(0.5, 20.0, 60))
    p, Ap, _, status = steihaug_cg(lambda v: A @ v, b, 1e6, tol=1e-10, max_iter=200)
    assert status == "converged"
    assert float((p - torch.linalg.solve(A, b)).abs().max()) <= 1e-7
    assert float((Ap - A @ p).abs().max()) <= 1e-9 * float(Ap.abs().max())
    p, Ap, _, status = steihaug_cg(lambda v: A @ v, b, 0.05, tol=1e-10, max_iter=200)
    assert status == "boundary" and math.isclose(float(torch.linalg.vector_norm(p)), 0.05, rel_tol=1e-9)
    assert float((Ap - A @ p).abs().max()) <= 1e-9 * float(Ap.abs().max())
    H, _ = _spectral(np.concatenate([[-1.0], np.linspace(0.2, 10.0, 59)]))
    p, Ap, _, status = steihaug_cg(lambda v: H @ v, b, 2.0, tol=1e-12, max_iter=200)
    assert status in ("neg_curv", "boundary") and math.isclose(float(torch.linalg.vector_norm(p)), 2.0, rel_tol=1e-9)
    # model decrease: -b^T p + p^T H p / 2 < 0 (the step improves the quadratic model)
    assert -float(b @ p) + 0.5 * float(p @ (H @ p)) < 0.0


def test_lanczos_extremes_and_min_eigpair():
    lams = np.concatenate([[-2.0, -1.5], np.linspace(0.1, 5.0, 56), [9.0, 12.0]])
    A, Q = _spectral(lams, seed=3)
    lo, hi = lanczos_extremes(lambda v: A @ v, 60, m=12, device="cpu")
    assert math.isclose(hi, 12.0, rel_tol=1e-6)           # the top edge converges within a few steps
    lo, hi = lanczos_extremes(lambda v: A @ v, 60, m=60, device="cpu")
    assert math.isclose(lo, -2.0, rel_tol=1e-8) and math.isclose(hi, 12.0, rel_tol=1e-8)
    lam, v = lanczos_min_eigpair(lambda v: A @ v, 60, m=60, device="cpu")
    assert math.isclose(lam, -2.0, rel_tol=1e-8)
    assert float(torch.linalg.vector_norm(A @ v - lam * v)) <= 1e-6
    assert abs(abs(float(v @ Q[:, 0])) - 1.0) <= 1e-6     # the eigenvector of -2


class _Func:
    """f(x) = x^T A x / 2 - b^T x + c sum x^4 / 4 (strictly convex) with exact derivatives."""

    def __init__(self, n=12, c=0.5, seed=4, shift=0.0):
        A, _ = _spectral(np.linspace(0.5 + shift, 4.0 + shift, n), seed=seed)
        self.A, self.b, self.c = A, _rhs(n, seed + 1), c
        self.shape = (n,)
        self.evals = 0

    def value(self, x):
        return float(0.5 * x @ (self.A @ x) - self.b @ x + 0.25 * self.c * (x ** 4).sum())

    def value_and_grad(self, x):
        self.evals += 1
        return self.value(x), self.A @ x - self.b + self.c * x ** 3

    def hvp(self, x, kind):
        assert kind in ("exact", "ggn", "fd_hessian")
        return lambda v: self.A @ v + 3.0 * self.c * x ** 2 * v


@pytest.mark.parametrize("driver", ["newton_cg", "newton_tr", "newton_lanczos"])
def test_drivers_reach_the_minimiser(driver):
    f = _Func()
    x0 = torch.zeros(12, dtype=torch.float64) + 3.0
    kw = dict(objective=f, verbose=False, gtol=1e-9)
    if driver == "newton_cg":
        x, hist = newton_cg(None, x0, None, curvature="exact", lam0=1e-3, max_newton=40, **kw)
    elif driver == "newton_tr":
        x, hist = newton_tr(None, x0, None, curvature="exact", delta0=0.5, max_newton=60, **kw)
    else:
        x, hist = newton_lanczos(None, x0, None, curvature="exact", sigma=1e-3, sigma_floor=1e-8, max_newton=60,
                                 lanczos_m=12, **kw)
    _, g = f.value_and_grad(x)
    assert float(torch.linalg.vector_norm(g)) <= 1e-7, hist[-3:]
    losses = [h["loss"] for h in hist]
    assert all(b <= a + 1e-12 for a, b in zip(losses, losses[1:]))  # accepted steps only decrease the loss


def test_trust_region_leaves_a_saddle():
    """f(x) = sum (x_i^2 - 1)^2 + 0.1 x_0: from the saddle at 0 the trust region follows negative curvature."""

    class Saddle:
        shape = (4,)
        evals = 0

        def value(self, x):
            return float(((x ** 2 - 1) ** 2).sum() + 0.1 * x[0])

        def value_and_grad(self, x):
            g = 4 * x * (x ** 2 - 1)
            g[0] += 0.1
            return self.value(x), g

        def hvp(self, x, kind):
            return lambda v: (12 * x ** 2 - 4) * v

    x0 = torch.full((4,), 1e-3, dtype=torch.float64)
    x, hist = newton_tr(None, x0, None, objective=Saddle(), gtol=1e-8, delta0=0.5, max_newton=60, verbose=False)
    assert torch.allclose(x.abs(), torch.ones(4, dtype=torch.float64), atol=0.06)
    assert Saddle().value(x) < Saddle().value(x0) - 1.0
