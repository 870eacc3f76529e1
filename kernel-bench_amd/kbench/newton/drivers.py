"""Newton-type drivers over the solve: damped Newton-CG, Steihaug trust region, Lanczos / witness Newton.

Same entry points, options and step rules as the reference's
newton/newton_cg.py (``newton_cg`` 302-392, ``newton_tr`` 220-299,
``newton_lanczos`` 47-217): each step evaluates the loss and gradient at
theta, solves a curvature system matrix-free with the Krylov solvers of
``kbench.newton.krylov``, and globalises the step (Armijo backtracking on the
loss, or the trust-region ratio test).

The loss and gradient come from an ``Objective``: by default the native
whole-pass driver (``kbench.runtime``, a few ms per evaluation at config 3).
Curvature is a named provider of the objective, built at the current point:
``"ggn"`` (the Gauss-Newton product, the default of ``newton_cg`` as in the
reference), ``"exact"`` (the exact Hessian-vector product) -- both from
``kbench.newton.hvp`` over the per-call wrappers -- and ``"fd_hessian"``
(central differences of two native gradients along the unit direction).  A
caller may add or replace providers (``curvatures=``).
Newton vectors are float64; theta is evaluated in float32.  The forward is not
warm-started from the previous E (the native E fixed point starts at e_init).
"""

from __future__ import annotations

import math

import torch

from .krylov import cg_solve, cg_witness, lanczos_extremes, steihaug_cg


class Objective:
    """The summed loss of one static problem as a function of flat theta vectors.

    ``curvatures`` maps a name to ``factory(objective, x) -> hvp`` (``hvp(v)`` of
    flat float64 vectors); ``"ggn"``, ``"exact"`` and ``"fd_hessian"`` are always
    available.  The first two evaluate the forward at x and build the product there
    (``make_ggn_hvp`` / ``make_exact_hvp``; uniform column weights).  The step
    ``fd_eps`` trades the float32 gradient's rounding (large for small steps)
    against the O(step^2) truncation: at config 1 a step of 1e-2 agrees with
    the exact HVP to 2e-3 (1e-3 only to 4e-2).
    """

    def __init__(self, static, col_weights, *, curvatures=None, fd_eps=1e-2):
        from kbench.runtime import fused_solver

        self.static = static
        self.col_weights = col_weights
        self.solver = fused_solver(static)
        S = int(static.state_helpers["S"])
        self.shape = (S, 3) if static.statewise else (3,)
        self.fd_eps = float(fd_eps)
        self.evals = 0   # loss + gradient evaluations
        self.values = 0  # loss-only evaluations
        self.curvatures = {"ggn": _ggn, "exact": _exact, "fd_hessian": _fd_hessian, **(curvatures or {})}

    def theta(self, x):
        return x.to(torch.float32).reshape(self.shape).contiguous()

    def value(self, x) -> float:
        self.values += 1
        with torch.no_grad():
            loss, _ = self.solver.run_forward(self.theta(x), self.col_weights)
        return float(loss)

    def value_and_grad(self, x):
        self.evals += 1
        th = self.theta(x)
        with torch.no_grad():
            loss, _, g, _ = self.solver.solve(th, self.col_weights)
        return float(loss), g.reshape(-1).double()

    def hvp(self, x, kind: str):
        if kind not in self.curvatures:
            raise ValueError(f"unknown curvature {kind!r}; available: {sorted(self.curvatures)}")
        return self.curvatures[kind](self, x)


def _at_point(obj: Objective, x):
    """(theta, forward intermediates) at x, from the whole-pass forward."""
    th = obj.theta(x)
    with torch.no_grad():
        _, saved = obj.solver.run_forward(th, obj.col_weights)
    saved.pop("_use_col_weights", None)
    return th, saved


def _ggn(obj: Objective, x):
    """The Gauss-Newton product at x (reference newton_cg.py:351-352 -> ggn.py:280)."""
    from .hvp import make_ggn_hvp

    th, saved = _at_point(obj, x)
    return make_ggn_hvp(obj.static, th, obj.col_weights, saved)


def _exact(obj: Objective, x):
    """The exact Hessian-vector product at x (reference hvp_exact.py:66)."""
    from .hvp import make_exact_hvp

    th, saved = _at_point(obj, x)
    return make_exact_hvp(obj.static, th, obj.col_weights, saved)


def _fd_hessian(obj: Objective, x):
    """H v by central differences of the gradient along v / ||v|| (step ``obj.fd_eps``)."""
    base = x.double()

    def hvp(v):
        v = v.double()
        nv = float(torch.linalg.vector_norm(v))
        if nv == 0.0:
            return torch.zeros_like(v)
        u = v / nv
        _, gp = obj.value_and_grad(base + obj.fd_eps * u)
        _, gm = obj.value_and_grad(base - obj.fd_eps * u)
        return nv * (gp - gm) / (2.0 * obj.fd_eps)

    return hvp


def _objective(static, col_weights, objective):
    return objective if objective is not None else Objective(static, col_weights)


def _armijo(value, x, p, F, slope, *, c1, tries):
    """Backtracking from alpha = 1 until value(x + alpha p) <= F + c1 alpha slope -> (alpha, value) or (None, None)."""
    alpha = 1.0
    for _ in range(int(tries)):
        Ft = value(x + alpha * p)
        if Ft <= F + c1 * alpha * slope:
            return alpha, Ft
        alpha *= 0.5
    return None, None


def _say(verbose, msg, end="\n"):
    if verbose:
        print(msg, end=end, flush=True)


def newton_cg(static, theta0, col_weights, *, curvature="ggn", max_newton=25, gtol=1e-2, lam0=1.0, lam_min=1e-7,
              lam_max=1e10, max_cg=30, eta_max=0.1, c1=1e-4, ls_max=25, objective=None, verbose=True):
    """Levenberg-Marquardt damped Newton-CG -> (theta, history) (reference newton_cg.py:302-392).

    Each step solves (H + lam I) p = -g by CG to tol eta ||g|| with eta =
    min(eta_max, sqrt ||g||), falls back to -g if p is not a descent direction,
    and backtracks; lam shrinks by 0.4 after a full step, grows by 1.5 after a
    shortened one and by 8 after a failed line search.
    """
    obj = _objective(static, col_weights, objective)
    x = theta0.reshape(-1).double().clone()
    lam = float(lam0)
    history = []
    for k in range(int(max_newton)):
        loss, g = obj.value_and_grad(x)
        gnorm = float(torch.linalg.vector_norm(g))
        history.append({"newton": k, "loss": loss, "gnorm": gnorm, "lam": lam})
        _say(verbose, f"[newton {k:2d}] loss={loss:.6f}  ||g||={gnorm:.4e}  lam={lam:.2e}", end="")
        if gnorm < gtol:
            _say(verbose, "  converged")
            break
        H = obj.hvp(x, curvature)
        eta = min(eta_max, math.sqrt(gnorm))
        p, iters, ok = cg_solve(lambda v: H(v).double() + lam * v, -g, tol=eta * gnorm, max_iter=max_cg)
        slope = float(torch.dot(g, p))
        if slope >= 0.0:
            p, slope = -g, -gnorm * gnorm
        alpha, Ft = _armijo(obj.value, x, p, loss, slope, c1=c1, tries=ls_max)
        history[-1].update(cg=iters, cg_converged=ok, alpha=alpha)
        if alpha is not None:
            x = x + alpha * p
            lam = max(lam_min, lam * (0.4 if alpha == 1.0 else 1.5))
            _say(verbose, f"  cg={iters}{'' if ok else '*'}  a={alpha:.2e}  d_loss={Ft - loss:+.4e}")
        else:
            lam = min(lam_max, 8.0 * lam)
            _say(verbose, f"  cg={iters}  line-search failed -> lam={lam:.2e}")
            if lam >= lam_max:
                break
    return x.reshape(obj.shape), history


def newton_tr(static, theta0, col_weights, *, curvature="fd_hessian", max_newton=30, gtol=1e-2, delta0=1.0,
              delta_max=1e3, eta_accept=0.05, max_cg=40, lam=0.0, theta_ref=None, objective=None, verbose=True):
    """Steihaug trust-region Newton -> (theta, history) (reference newton_cg.py:220-299).

    Minimises F = L + lam/2 ||x - theta_ref||^2 (theta_ref defaults to theta0).
    The radius shrinks to ||p|| / 4 when the actual / predicted reduction
    ratio is below 1/4, doubles (up to delta_max) above 3/4 with a boundary
    step; a step is accepted when the ratio exceeds eta_accept and F
    decreased.  Three rejections in a row, or a collapsed radius, stop.
    """
    obj = _objective(static, col_weights, objective)
    x = theta0.reshape(-1).double().clone()
    ref = (x if theta_ref is None else theta_ref.reshape(-1).double()).clone()
    lam = float(lam)
    penalty = (lambda z: 0.5 * lam * float(torch.sum((z - ref) ** 2))) if lam > 0 else (lambda z: 0.0)
    delta = float(delta0)
    history = []
    rejects = 0
    loss, g = obj.value_and_grad(x)
    for k in range(int(max_newton)):
        gF = g + lam * (x - ref) if lam > 0 else g
        F = loss + penalty(x)
        gnorm = float(torch.linalg.vector_norm(gF))
        history.append({"newton": k, "loss": loss, "F": F, "gnorm": gnorm, "delta": delta})
        _say(verbose, f"[tr {k:2d}] F={F:.6f}  ||gF||={gnorm:.4e}  delta={delta:.2e}", end="")
        if gnorm < gtol:
            _say(verbose, "  converged")
            break
        H = obj.hvp(x, curvature)
        op = (lambda v: H(v).double() + lam * v) if lam > 0 else (lambda v: H(v).double())
        p, Ap, iters, status = steihaug_cg(op, -gF, delta, tol=min(0.1, math.sqrt(gnorm)) * gnorm, max_iter=max_cg)
        pred = -float(torch.dot(gF, p)) - 0.5 * float(torch.dot(p, Ap))
        pnorm = float(torch.linalg.vector_norm(p))
        trial = x + p
        Ft = obj.value(trial) + penalty(trial)
        ared = F - Ft
        rho = ared / pred if pred > 0 else -1.0
        if rho < 0.25:
            delta = 0.25 * pnorm
        elif rho > 0.75 and pnorm >= 0.99 * delta:
            delta = min(2.0 * delta, delta_max)
        history[-1].update(cg=iters, status=status, rho=rho, step=pnorm)
        if rho > eta_accept and ared > 0:
            rejects = 0
            x = trial
            _say(verbose, f"  cg={iters}({status})  |p|={pnorm:.2e}  rho={rho:.2f}  dF={-ared:+.4e}")
            loss, g = obj.value_and_grad(x)
        else:
            rejects += 1
            _say(verbose, f"  cg={iters}({status})  |p|={pnorm:.2e}  rho={rho:.2f}  REJECT")
            if delta < 1e-10 or rejects >= 3:
                break
    return x.reshape(obj.shape), history


def newton_lanczos(static, theta0, col_weights, *, sigma=0.01, sigma_floor=1e-4, lanczos_m=10, nu=1.5, omega=1.5,
                   max_bumps=3, eta_max=0.1, max_cg=40, c1=1e-4, ls_max=25, gtol=1e-2, max_newton=40, lam=0.0,
                   theta_ref=None, lanczos_refresh=0, ftol=1e-9, curvature="fd_hessian", objective=None,
                   verbose=True):
    """Lanczos-initialised, witness-corrected damped Newton -> (theta, history) (reference newton_cg.py:47-217).

    The damping starts at sigma * lambda_max (m-step Lanczos), with floor
    sigma_floor * lambda_max and ceiling 10 * lambda_max.  When CG on
    H + lam_damp I meets non-positive curvature its certificate c raises the
    damping to nu (lam_damp - c) and the solve restarts (at most max_bumps
    times, then a scaled gradient step).  Armijo backtracking on
    F = L + lam/2 ||x - theta_ref||^2; the damping shrinks by omega after a
    full step, grows by 1.5 after a shortened one and by 4 after a failed
    search; two accepted improvements below ftol in a row stop.
    """
    obj = _objective(static, col_weights, objective)
    x = theta0.reshape(-1).double().clone()
    n = x.numel()
    ref = (x if theta_ref is None else theta_ref.reshape(-1).double()).clone()
    lam = float(lam)
    penalty = (lambda z: 0.5 * lam * float(torch.sum((z - ref) ** 2))) if lam > 0 else (lambda z: 0.0)
    value_F = lambda z: obj.value(z) + penalty(z)  # noqa: E731

    def curvature_at(z):
        H = obj.hvp(z, curvature)
        return (lambda v: H(v).double() + lam * v) if lam > 0 else (lambda v: H(v).double())

    loss, g = obj.value_and_grad(x)
    H = curvature_at(x)
    _, top = lanczos_extremes(H, n, m=lanczos_m, device=str(x.device))
    damp, floor, ceil = sigma * top, sigma_floor * top, 10.0 * top
    _say(verbose, f"[lanczos-newton] m={lanczos_m}  lam_max~{top:.2f}  lam_damp0={damp:.4f}")
    history = []
    accepted = stalls = 0
    stale = False
    for k in range(int(max_newton)):
        gF = g + lam * (x - ref) if lam > 0 else g
        F = loss + penalty(x)
        gnorm = float(torch.linalg.vector_norm(gF))
        rec = {"newton": k, "loss": loss, "F": F, "gnorm": gnorm, "lam_damp": damp, "witness_certs": [],
               "evals": obj.evals}
        history.append(rec)
        _say(verbose, f"[ln {k:2d}] F={F:.6f}  ||gF||={gnorm:.4e}  lam={damp:.3e}", end="")
        if gnorm < gtol:
            _say(verbose, "  converged")
            break
        refresh = bool(lanczos_refresh and accepted and accepted % int(lanczos_refresh) == 0)
        if stale or refresh:
            H = curvature_at(x)
            stale = False
            if refresh:
                _, top = lanczos_extremes(H, n, m=lanczos_m, device=str(x.device))
                floor, ceil = sigma_floor * top, 10.0 * top
        eta = min(eta_max, math.sqrt(gnorm))
        status, p, iters = "", None, 0
        for _ in range(int(max_bumps) + 1):
            p, iters, status, cert = cg_witness(lambda v: H(v) + damp * v, -gF, tol=eta * gnorm, max_iter=max_cg)
            if status != "neg_curv":
                break
            rec["witness_certs"].append(damp - cert)
            damp = min(ceil, nu * (damp - cert))
        if status == "neg_curv":
            p, status = -gF / damp, "fallback_gd"
        slope = float(torch.dot(gF, p))
        if slope >= 0.0:
            p, slope, status = -gF / damp, -gnorm * gnorm / damp, status + "+gd"
        rec.update(cg=iters, status=status)
        alpha, Ft = _armijo(value_F, x, p, F, slope, c1=c1, tries=ls_max)
        rec["alpha"] = alpha
        if alpha is not None:
            accepted += 1
            x = x + alpha * p
            stale = True
            damp = max(floor, damp / omega) if alpha == 1.0 else min(ceil, 1.5 * damp)
            _say(verbose, f"  cg={iters}({status})  a={alpha:.2e}  dF={Ft - F:+.4e}")
            stalls = stalls + 1 if (F - Ft) <= ftol * max(1.0, abs(F)) else 0
            if stalls >= 2:
                break
            loss, g = obj.value_and_grad(x)
        else:
            damp = min(ceil, 4.0 * damp)
            _say(verbose, f"  cg={iters}({status})  line-search failed -> lam={damp:.3e}")
            if damp >= ceil:
                break
    return x.reshape(obj.shape), history
