"""Newton drivers on the real solve (config 1, per-species theta) with the native objective.

The loss and gradient come from the native whole-pass driver; curvature from
the package's exact and Gauss-Newton HVPs (``kbench.newton.hvp``, pinned
against the oracle in tests/test_hvp_gpu.py) or from central differences of
native gradients (``fd_hessian``).  Checked: the FD product agrees with the
exact one; ``newton_cg`` runs with its defaults (Gauss-Newton curvature);
Newton-CG on the HIP objective takes the steps that the same driver takes
over the float64 oracle's loss, gradient and exact HVP; and a few steps of
each driver decrease the loss.
"""

import numpy as np
import pytest
import torch

import kbench_oracle as O
import kbtest

pytestmark = pytest.mark.gpu


def _setup():
    from kbench import percall
    from kbench.fused import problem_to_captured
    from kbench.newton import Objective
    from kbench.newton.hvp import make_exact_hvp
    from kbench.runtime import make_static

    c0 = problem_to_captured(kbtest.problem("1", True))
    static = make_static(c0, "cuda")
    theta, cw = c0["inputs"]["theta"].cuda(), c0["inputs"]["col_weights"].cuda()

    def exact_rows(obj, x):  # every row computed, no graph
        th = obj.theta(x)
        _, sv = percall.run_forward(static, th, cw)
        return make_exact_hvp(static, th, cw, sv, row_classes=False, graph=False)

    obj = Objective(static, cw, curvatures={"exact_rows": exact_rows})
    return static, theta, cw, obj


class OracleObjective:
    """The float64 oracle's loss, gradient and exact HVP at the float32-rounded point x, with the
    interface the Newton drivers call (``value``, ``value_and_grad``, ``hvp``)."""

    def __init__(self, name, statewise):
        p = kbtest.problem(name, statewise)
        self.prob = O.Problem.from_dict(p)
        self.cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
        self.shape = np.asarray(p["inputs"]["theta"]).shape

    def _th(self, x):
        return x.detach().cpu().numpy().astype(np.float32).astype(np.float64).reshape(self.shape)

    def value(self, x) -> float:
        loss, _ = O.forward(self.prob, self._th(x), self.cw)
        return float(loss)

    def value_and_grad(self, x):
        th = self._th(x)
        loss, saved = O.forward(self.prob, th, self.cw)
        gt, _, _ = O.backward(self.prob, th, self.cw, saved)
        return float(loss), torch.as_tensor(gt.reshape(-1), dtype=torch.float64, device=x.device)

    def hvp(self, x, kind):
        assert kind == "exact", kind
        th = self._th(x)
        _, saved = O.forward(self.prob, th, self.cw)
        _, _, cache = O.build_point_cache(self.prob, th, self.cw, saved)
        return lambda v: torch.as_tensor(O.hvp_exact(self.prob, th, saved, v.detach().cpu().numpy().reshape(
            self.shape), cache).reshape(-1), dtype=torch.float64, device=v.device)


def Objective_default_eps():
    import inspect

    from kbench.newton import Objective

    return inspect.signature(Objective).parameters["fd_eps"].default


def test_fd_hessian_agrees_with_the_exact_hvp():
    print("[newton] fd_hessian vs exact HVP, config=1 statewise", flush=True)
    static, theta, cw, obj = _setup()
    x = theta.reshape(-1).double()
    v = torch.as_tensor(np.random.default_rng(9).normal(size=x.numel()), dtype=torch.float64, device="cuda")
    ex = obj.hvp(x, "exact")(v).double()
    rels = {}
    for eps in (3e-2, 1e-2, 3e-3, 1e-3):
        obj.fd_eps = eps
        fd = obj.hvp(x, "fd_hessian")(v)
        rels[eps] = float((fd - ex).abs().max()) / float(ex.abs().max())
    torch.cuda.synchronize()
    print(f"  |H v|={float(ex.abs().max()):.4e}  fd vs exact rel by step: {rels}")
    assert rels[Objective_default_eps()] <= 5e-3


def test_newton_cg_steps_on_the_fast_hvp_match_the_row_by_row_ones():
    """Newton-CG on the class / graph HVP (the package default; a new point, so a new capture, every step)
    takes the steps the row-by-row HVP gives, to float32 rounding of the CG iterates."""
    from kbench import newton

    print("[newton] newton_cg exact vs exact_rows, config=1 statewise", flush=True)
    static, theta, cw, obj = _setup()
    out = {}
    for curv in ("exact_rows", "exact"):
        x, _ = newton.newton_cg(static, theta, cw, curvature=curv, objective=obj, max_newton=3, gtol=1e-12,
                                max_cg=20)
        out[curv] = x.reshape(-1).double()
    torch.cuda.synchronize()
    e = float((out["exact"] - out["exact_rows"]).abs().max()) / float(out["exact_rows"].abs().max())
    print(f"  x after 3 steps: rel diff {e:.3e}")
    assert e <= 1e-4


def test_newton_cg_runs_with_its_defaults():
    """``newton_cg(static, theta, cw)`` as a caller of the reference makes it (newton_cg.py:323): the
    default curvature is the Gauss-Newton product, built at every step by the package."""
    from kbench import newton

    print("[newton] newton_cg defaults (ggn), config=1 statewise", flush=True)
    static, theta, cw, _ = _setup()
    x, hist = newton.newton_cg(static, theta, cw, max_newton=3)
    torch.cuda.synchronize()
    print(f"  losses {[round(h['loss'], 6) for h in hist]}")
    assert len(hist) == 3 and all("cg" in h for h in hist)
    assert hist[-1]["loss"] < hist[0]["loss"]
    assert tuple(x.shape) == tuple(theta.shape)


def test_newton_cg_matches_the_same_driver_over_the_oracle():
    """Three Newton-CG steps with exact curvature on the HIP objective and on the float64 oracle's
    objective (loss, gradient and ``O.hvp_exact`` at the same float32 points; reference
    newton/newton_cg.py:302-392 with hvp_exact.py).  CG runs a fixed 5 iterations (eta_max 1e-12), so
    both sides take the same discrete decisions; iterates agree to rel 1e-4, losses to 1e-6."""
    from kbench import newton

    print("[newton] newton_cg exact: HIP objective vs oracle objective, config=1 statewise", flush=True)
    static, theta, cw, obj = _setup()
    kw = dict(curvature="exact", max_newton=3, gtol=1e-12, max_cg=5, eta_max=1e-12, verbose=True)
    x_h, hist_h = newton.newton_cg(static, theta, cw, objective=obj, **kw)
    x_o, hist_o = newton.newton_cg(static, theta, cw, objective=OracleObjective("1", True), **kw)
    torch.cuda.synchronize()
    xh, xo = x_h.reshape(-1).double(), x_o.reshape(-1).double()
    e = float((xh - xo).abs().max()) / float(xo.abs().max())
    print(f"  iterates rel={e:.3e}")
    for a, b in zip(hist_h, hist_o):
        rl = abs(a["loss"] - b["loss"]) / abs(b["loss"])
        print(f"  step {a['newton']}: loss hip={a['loss']:.9f} oracle={b['loss']:.9f} rel={rl:.2e} "
              f"cg={a.get('cg')}/{b.get('cg')} alpha={a.get('alpha')}/{b.get('alpha')}")
        assert rl <= 1e-6
        assert a.get("cg") == b.get("cg") and a.get("alpha") == b.get("alpha")
    assert e <= 1e-4


@pytest.mark.parametrize("driver,curv", [("newton_cg", "exact"), ("newton_cg", "exact_rows"), ("newton_cg", "ggn"),
                                         ("newton_tr", "fd_hessian"), ("newton_lanczos", "fd_hessian")])
def test_driver_steps_decrease_the_loss(driver, curv):
    from kbench import newton

    print(f"[newton] {driver} curvature={curv}, config=1 statewise", flush=True)
    static, theta, cw, obj = _setup()
    fn = getattr(newton, driver)
    kw = dict(curvature=curv, objective=obj, max_newton=3, gtol=1e-12, verbose=True)
    if driver == "newton_cg":
        kw.update(max_cg=20)
    elif driver == "newton_tr":
        kw.update(max_cg=20, delta0=0.5)
    else:
        kw.update(max_cg=20, lanczos_m=6)
    x, hist = fn(static, theta, cw, **kw)
    torch.cuda.synchronize()
    l0, g0 = obj.value_and_grad(theta.reshape(-1).double())
    l1, g1 = obj.value_and_grad(x.reshape(-1))
    print(f"  loss {l0:.6f} -> {l1:.6f}, |g| {float(g0.norm()):.4e} -> {float(g1.norm()):.4e}, "
          f"{obj.evals} gradient evaluations")
    assert l1 < l0  # (Armijo accepts only decreasing steps; the gradient norm need not fall every step)
