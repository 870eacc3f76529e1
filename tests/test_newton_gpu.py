"""Newton drivers on the real solve (config 1, per-species theta) with the native objective.

The loss and gradient come from the native whole-pass driver; curvature from
central differences of native gradients (``fd_hessian``), or from the exact /
Gauss-Newton HVPs of the per-call wrapper path (pinned against the oracle in
tests/test_hvp_gpu.py).  Checked: the FD product agrees with the exact one,
and a few steps of each driver decrease the loss and the gradient norm.
"""

import numpy as np
import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


def _setup():
    import dropin
    from dropin.hvp import HvpPlan, ggn_hvp
    from dropin.solve import plan_of
    from kbench.fused import problem_to_captured
    from kbench.newton import Objective
    from kbench.runtime import make_static

    c0 = problem_to_captured(kbtest.problem("1", True))
    static = make_static(c0, "cuda")
    theta, cw = c0["inputs"]["theta"].cuda(), c0["inputs"]["col_weights"].cuda()

    def exact(obj, x):
        th = obj.theta(x)
        _, sv = dropin.run_forward(static, th, cw)
        return HvpPlan(plan_of(static), th, cw, sv)

    def exact_classes(obj, x):  # the fast HVP: row classes, tangent passes replayed as one graph
        th = obj.theta(x)
        _, sv = dropin.run_forward(static, th, cw)
        return HvpPlan(plan_of(static), th, cw, sv, row_classes=True, graph=True)

    def ggn(obj, x):
        th = obj.theta(x)
        _, sv = dropin.run_forward(static, th, cw)
        return ggn_hvp(plan_of(static), th, cw, sv)

    obj = Objective(static, cw, curvatures={"exact": exact, "exact_classes": exact_classes, "ggn": ggn})
    return static, theta, cw, obj


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
    """Newton-CG on the class / graph HVP (a new point, so a new capture, every step) takes the steps the
    row-by-row HVP gives, to float32 rounding of the CG iterates."""
    from kbench import newton

    print("[newton] newton_cg exact vs exact_classes, config=1 statewise", flush=True)
    static, theta, cw, obj = _setup()
    out = {}
    for curv in ("exact", "exact_classes"):
        x, _ = newton.newton_cg(static, theta, cw, curvature=curv, objective=obj, max_newton=3, gtol=1e-12,
                                max_cg=20)
        out[curv] = x.reshape(-1).double()
    torch.cuda.synchronize()
    e = float((out["exact_classes"] - out["exact"]).abs().max()) / float(out["exact"].abs().max())
    print(f"  x after 3 steps: rel diff {e:.3e}")
    assert e <= 1e-4


@pytest.mark.parametrize("driver,curv", [("newton_cg", "exact"), ("newton_cg", "exact_classes"), ("newton_cg", "ggn"),
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
