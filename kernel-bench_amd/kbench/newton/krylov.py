"""Matrix-free Krylov solvers for the Newton drivers (reference newton/cg.py:13-182).

Every operator is a callable ``apply(v) -> A v`` on flat float64 vectors, so a
Hessian-vector product from any source plugs in.  Scalars are host floats.

* ``cg_solve``: conjugate gradients, stops on ||r|| <= tol;
* ``cg_witness``: CG that stops at the first direction of non-positive
  curvature and returns its Rayleigh quotient d^T A d / ||d||^2 as a
  certificate (with A = H + lam I it proves lambda_min(H) <= cert - lam);
* ``steihaug_cg``: truncated CG for the trust-region subproblem
  min -b^T p + p^T A p / 2 s.t. ||p|| <= delta (Steihaug 1983, Toint 1981),
  following negative curvature to the boundary; returns A p as accumulated
  from the iteration's products (no extra operator call);
* ``lanczos_extremes`` / ``lanczos_min_eigpair``: m-step Lanczos with full
  reorthogonalisation, extremal Ritz values (and the smallest Ritz vector).
"""

from __future__ import annotations

import math

import torch


def _dot(a, b) -> float:
    return float(torch.dot(a, b))


def cg_solve(apply, b, *, tol, max_iter, x0=None):
    """Solve A x = b (A symmetric positive definite) -> (x, iterations, converged)."""
    x = torch.zeros_like(b) if x0 is None else x0.clone()
    r = b.clone() if x0 is None else b - apply(x)
    if _dot(b, b) == 0.0:
        return x, 0, True
    d = r.clone()
    rr = _dot(r, r)
    it = 0
    for it in range(1, int(max_iter) + 1):
        Ad = apply(d)
        curv = _dot(d, Ad)
        if curv <= 0.0:  # not positive definite along d: keep the last iterate
            if it == 1:  # (a first step along b scaled by the curvature magnitude, else b)
                x = b / max(curv / max(_dot(d, d), 1e-30), 1e-12) if curv != 0.0 else b
            break
        step = rr / curv
        x = x + step * d
        r = r - step * Ad
        rr_next = _dot(r, r)
        if math.sqrt(rr_next) <= tol:
            return x, it, True
        d = r + (rr_next / rr) * d
        rr = rr_next
    return x, it, False


def cg_witness(apply, b, *, tol, max_iter):
    """CG reporting negative curvature -> (x, iterations, status, certificate).

    status: 'converged', 'max_iter' or 'neg_curv'; the certificate (None unless
    'neg_curv') is d^T A d / ||d||^2 <= 0 of the offending direction d.
    """
    x = torch.zeros_like(b)
    r = b.clone()
    d = r.clone()
    rr = _dot(r, r)
    if math.sqrt(rr) <= tol:
        return x, 0, "converged", None
    for it in range(1, int(max_iter) + 1):
        Ad = apply(d)
        curv = _dot(d, Ad)
        if curv <= 0.0:
            return x, it, "neg_curv", curv / _dot(d, d)
        step = rr / curv
        x = x + step * d
        r = r - step * Ad
        rr_next = _dot(r, r)
        if math.sqrt(rr_next) <= tol:
            return x, it, "converged", None
        d = r + (rr_next / rr) * d
        rr = rr_next
    return x, int(max_iter), "max_iter", None


def _to_sphere(p, d, radius) -> float:
    """The tau > 0 with ||p + tau d|| = radius (||p|| < radius)."""
    pd, dd, pp = _dot(p, d), _dot(d, d), _dot(p, p)
    return (-pd + math.sqrt(pd * pd + dd * (radius * radius - pp))) / dd


def steihaug_cg(apply, b, delta, *, tol, max_iter):
    """Trust-region CG -> (p, A p, iterations, status).

    status: 'converged', 'boundary' (the step reached ||p|| = delta), 'neg_curv'
    (a non-positive curvature direction was followed to the boundary) or 'max_iter'.
    """
    p = torch.zeros_like(b)
    Ap = torch.zeros_like(b)
    r = b.clone()
    d = r.clone()
    rr = _dot(r, r)
    if math.sqrt(rr) <= tol:
        return p, Ap, 0, "converged"
    for it in range(1, int(max_iter) + 1):
        Ad = apply(d)
        curv = _dot(d, Ad)
        if curv <= 0.0:
            tau = _to_sphere(p, d, delta)
            return p + tau * d, Ap + tau * Ad, it, "neg_curv"
        step = rr / curv
        nxt = p + step * d
        if float(torch.linalg.vector_norm(nxt)) >= delta:
            tau = _to_sphere(p, d, delta)
            return p + tau * d, Ap + tau * Ad, it, "boundary"
        p, Ap = nxt, Ap + step * Ad
        r = r - step * Ad
        rr_next = _dot(r, r)
        if math.sqrt(rr_next) <= tol:
            return p, Ap, it, "converged"
        d = r + (rr_next / rr) * d
        rr = rr_next
    return p, Ap, int(max_iter), "max_iter"


def lanczos(apply, n, *, m, seed=0, device="cuda", dtype=torch.float64):
    """m-step Lanczos with full reorthogonalisation from a seeded random start.

    Returns (Q, alpha, beta): the orthonormal basis vectors, the diagonal and the
    off-diagonal of the tridiagonal T = Q^T A Q (len(beta) = len(alpha) - 1
    unless the Krylov space closed early).
    """
    gen = torch.Generator(device=device).manual_seed(int(seed))
    q = torch.randn(int(n), generator=gen, device=device, dtype=dtype)
    q = q / torch.linalg.vector_norm(q)
    Q, alpha, beta = [], [], []
    q_prev, b_prev = torch.zeros_like(q), 0.0
    for _ in range(int(m)):
        w = apply(q) - b_prev * q_prev
        a = _dot(w, q)
        w = w - a * q
        for qi in Q:
            w = w - _dot(w, qi) * qi
        Q.append(q)
        alpha.append(a)
        b = float(torch.linalg.vector_norm(w))
        if b < 1e-12:
            break
        q_prev, q, b_prev = q, w / b, b
        beta.append(b)
    return Q, alpha, beta[: max(len(alpha) - 1, 0)]


def _ritz(alpha, beta, vectors: bool):
    import numpy as np
    from scipy.linalg import eigh_tridiagonal

    return eigh_tridiagonal(np.asarray(alpha), np.asarray(beta), eigvals_only=not vectors)


def lanczos_extremes(apply, n, *, m=40, seed=0, device="cuda", dtype=torch.float64):
    """(lambda_min, lambda_max) Ritz estimates after m Lanczos steps (lambda_min converges from above)."""
    _, alpha, beta = lanczos(apply, n, m=m, seed=seed, device=device, dtype=dtype)
    ev = _ritz(alpha, beta, vectors=False)
    return float(ev[0]), float(ev[-1])


def lanczos_min_eigpair(apply, n, *, m=120, seed=0, device="cuda", dtype=torch.float64):
    """(lambda_min, unit Ritz vector) after m Lanczos steps; check ||A v - lambda v|| before trusting v."""
    Q, alpha, beta = lanczos(apply, n, m=m, seed=seed, device=device, dtype=dtype)
    ev, S = _ritz(alpha, beta, vectors=True)
    s = torch.as_tensor(S[:, 0], device=device, dtype=dtype)
    v = torch.stack(Q).T @ s
    return float(ev[0]), v / torch.linalg.vector_norm(v)
