"""Unpreconditioned BiCGSTAB (van der Vorst, SIAM J. Sci. Stat. Comput. 13(2), 1992).

The reference solves its E adjoint with this method and fixes the stopping
and breakdown rules a caller observes (its kbench/api/_implicit_grad.py:28-94):

* residuals are relative to max(||b||, 1);
* the zero start is returned when its residual already meets ``tol``;
* after the half step s = r - alpha v the method stops on ||s|| (x + alpha p);
* a breakdown is a quantity at most ``breakdown_tol`` in magnitude among
  rho = <r0, r>, <r0, v>, <t, t> and omega (tested after the update);
* a breakdown, or ``max_iter`` full steps without convergence, raises
  RuntimeError.

The scalars are host floats (one device read per inner product).
"""

from __future__ import annotations

import torch


def _dot(a: torch.Tensor, b: torch.Tensor) -> float:
    return float(torch.dot(a, b))


def _nrm(a: torch.Tensor) -> float:
    return float(torch.linalg.vector_norm(a))


def bicgstab(apply, b: torch.Tensor, *, max_iter: int = 500, tol: float = 1e-7, breakdown_tol: float = 1e-30,
             info: dict | None = None) -> torch.Tensor:
    """Solve apply(x) = b for a flat vector b; ``info`` (optional) gets the step count and residual."""
    if int(max_iter) < 1 or not tol > 0.0 or not breakdown_tol > 0.0:
        raise ValueError("bicgstab needs max_iter >= 1 and positive tol / breakdown_tol")
    ref = max(_nrm(b), 1.0)
    x = torch.zeros_like(b)
    r = b - apply(x)
    res = _nrm(r) / ref
    steps = 0

    def done(sol):
        if info is not None:
            info.update(steps=steps, residual=res)
        return sol

    if res <= tol:
        return done(x)
    shadow = r.clone()
    p = torch.zeros_like(b)
    v = torch.zeros_like(b)
    rho_old = alpha = omega = 1.0
    while steps < int(max_iter):
        steps += 1
        rho = _dot(shadow, r)
        if abs(rho) <= breakdown_tol:
            break
        p = r + (rho / rho_old) * (alpha / omega) * (p - omega * v)
        v = apply(p)
        sv = _dot(shadow, v)
        if abs(sv) <= breakdown_tol:
            break
        alpha = rho / sv
        s = r - alpha * v
        res = _nrm(s) / ref
        if res <= tol:
            return done(x + alpha * p)
        t = apply(s)
        tt = _dot(t, t)
        if abs(tt) <= breakdown_tol:
            break
        omega = _dot(t, s) / tt
        x = x + alpha * p + omega * s
        r = s - omega * t
        res = _nrm(r) / ref
        if res <= tol:
            return done(x)
        if abs(omega) <= breakdown_tol:
            break
        rho_old = rho
    if info is not None:
        info.update(steps=steps, residual=res)
    raise RuntimeError(f"E-adjoint BiCGSTAB solve failed after {steps} iterations (relative residual {res:.3e})")
