"""Full-size GPU checks of the whole-pass driver (configs 3 and 4) and of its error contract.

At configs 3 and 4 the float64 oracle is too slow to run, so the native
whole-pass driver (``kbench.runtime`` / ``kbench.fused.FusedSolver``) is
checked through size-independent properties:

* it agrees with the per-call wrappers driven in the reference glue's call
  sequence (``dropin``), which the oracle pins on configs 1-2: loss rel
  <= 1e-5, identical -inf pattern of Pi / Pibar, Pi max_rel <= 1e-5 and
  max_abs <= 5e-3 (log2 units), gradients rel <= 1e-4 (max|diff| / max|ref|);
* repeated solves are bitwise identical (no atomics anywhere);
* computing one representative per class of identical rows (row classes) and
  computing every row (``KB_DEDUP=0``) agree: loss rel <= 1e-6, gradients rel
  <= 1e-5.

Error contract (reference kbench/api/_implicit_grad.py:94): a failed
E-adjoint BiCGSTAB raises RuntimeError; options the fused backward does not
implement raise; the driver's caches never match a different tensor that
reuses freed memory.
"""

import os

import numpy as np
import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


def _static(name, statewise=None, **opts):
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    p = kbtest.problem(name, statewise)
    cap = problem_to_captured(p)
    if opts:
        cap["meta"]["solver_options"] = dict(cap["meta"]["solver_options"], **opts)
    static = make_static(cap, "cuda")
    return static, cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()


def _free():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _forward_agrees(tag, s_fused, s_ref):
    for k in ("pi_wave", "pibar_wave", "pibar_row_max"):
        ok, ma, mr = kbtest.compare_inf_safe_t(s_fused[k], s_ref[k])
        print(f"  [{tag}] {k}: pattern={ok} max_abs={ma:.3e} max_rel={mr:.3e}", flush=True)
        assert ok, f"{k}: -inf pattern differs"
        # log2 values reach |x| ~ 1e3 at config 4, where one float32 ulp is 6e-5
        assert mr <= 1e-5 and ma <= 5e-3, f"{k}: max_abs {ma:.3e} max_rel {mr:.3e}"


def _fused_solve(solver, theta, cw):
    loss, saved = solver.run_forward(theta, cw)
    gt, gc = solver.run_backward(theta, cw, saved)
    return loss, saved, gt, gc


# ---------------------------------------------------------------------- config 3
def test_config3_fused_solve_matches_wrappers():
    """Config 3 (the bench workload): whole-pass forward + backward vs the per-call path."""
    from kbench import percall as dropin
    from kbench.runtime import fused_solver

    print("[fullsize] config=3 fused vs per-call wrappers (fwd + bwd)", flush=True)
    static, theta, cw = _static("3")
    l_ref, s_ref = dropin.run_forward(static, theta, cw)
    g_ref = dropin.run_backward(static, theta, cw, s_ref)
    loss, saved, gt, gc = _fused_solve(fused_solver(static), theta, cw)
    torch.cuda.synchronize()
    rel = abs(float(loss) - float(l_ref)) / abs(float(l_ref))
    print(f"  loss fused={float(loss):.9g} per-call={float(l_ref):.9g} rel={rel:.3e}")
    assert rel <= 1e-5
    _forward_agrees("config3", saved, s_ref)
    rt, rc = kbtest.norm_rel_t(gt, g_ref[0]), kbtest.norm_rel_t(gc, g_ref[1])
    print(f"  grad_theta rel={rt:.3e} grad_col rel={rc:.3e}")
    assert rt <= 1e-4 and rc <= 1e-4


def test_config3_fused_solve_is_bitwise_reproducible():
    from kbench.runtime import fused_solver

    print("[fullsize] config=3 fused run twice", flush=True)
    static, theta, cw = _static("3")
    solver = fused_solver(static)
    a = _fused_solve(solver, theta, cw)
    b = _fused_solve(solver, theta, cw)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0])
    for k in ("pi_wave", "pibar_wave", "pibar_row_max", "E"):
        assert torch.equal(a[1][k], b[1][k]), k
    assert torch.equal(a[2], b[2]) and torch.equal(a[3], b[3])


# ---------------------------------------------------------------------- config 4
@pytest.fixture(scope="module")
def config4():
    print("[fullsize] config=4 problem (S=8191, C=310757)", flush=True)
    out = _static("4")
    yield out
    _free()


def test_config4_fused_reproducible_and_row_classes_exact(config4):
    """Config 4: solve twice (bitwise), and row classes on vs off (KB_DEDUP=0)."""
    from kbench.fused import FusedSolver

    static, theta, cw = config4
    print("[fullsize] config=4 fused run twice + KB_DEDUP=0", flush=True)
    solver = FusedSolver(static, static.solver_options)
    a = _fused_solve(solver, theta, cw)
    b = _fused_solve(solver, theta, cw)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0])
    assert torch.equal(a[1]["pi_wave"], b[1]["pi_wave"]) and torch.equal(a[1]["pibar_wave"], b[1]["pibar_wave"])
    assert torch.equal(a[2], b[2]) and torch.equal(a[3], b[3])
    loss_a, gt_a, gc_a = a[0], a[2], a[3]
    del a, b, solver
    _free()
    old = os.environ.get("KB_DEDUP")
    os.environ["KB_DEDUP"] = "0"
    try:
        flat = FusedSolver(static, static.solver_options)  # the plan reads KB_DEDUP when it is created
    finally:
        if old is None:
            os.environ.pop("KB_DEDUP")
        else:
            os.environ["KB_DEDUP"] = old
    loss_b, _, gt_b, gc_b = _fused_solve(flat, theta, cw)
    torch.cuda.synchronize()
    rel = abs(float(loss_a) - float(loss_b)) / abs(float(loss_b))
    rt, rc = kbtest.norm_rel_t(gt_a, gt_b), kbtest.norm_rel_t(gc_a, gc_b)
    print(f"  dedup on/off: loss rel={rel:.3e} grad_theta rel={rt:.3e} grad_col rel={rc:.3e}")
    assert rel <= 1e-6 and rt <= 1e-5 and rc <= 1e-5
    del flat
    _free()


def test_config4_fused_solve_matches_wrappers(config4):
    """Config 4: whole-pass forward + backward vs the per-call path."""
    from kbench import percall as dropin
    from kbench.fused import FusedSolver

    static, theta, cw = config4
    print("[fullsize] config=4 fused vs per-call wrappers (fwd + bwd)", flush=True)
    solver = FusedSolver(static, static.solver_options)
    loss, saved, gt, gc = _fused_solve(solver, theta, cw)
    l_ref, s_ref = dropin.run_forward(static, theta, cw)
    torch.cuda.synchronize()
    rel = abs(float(loss) - float(l_ref)) / abs(float(l_ref))
    print(f"  loss fused={float(loss):.9g} per-call={float(l_ref):.9g} rel={rel:.3e}", flush=True)
    assert rel <= 1e-5
    _forward_agrees("config4", saved, s_ref)
    del saved, solver
    _free()
    g_ref = dropin.run_backward(static, theta, cw, s_ref)
    torch.cuda.synchronize()
    rt, rc = kbtest.norm_rel_t(gt, g_ref[0]), kbtest.norm_rel_t(gc, g_ref[1])
    print(f"  grad_theta rel={rt:.3e} grad_col rel={rc:.3e}")
    assert rt <= 1e-4 and rc <= 1e-4
    del s_ref, g_ref
    _free()


# ---------------------------------------------------------------------- error contract and caches
@pytest.mark.parametrize("path", ["fused", "per-call"])
def test_failed_e_adjoint_solve_raises(path):
    """One BiCGSTAB step at an unreachable tolerance: the backward raises RuntimeError (_implicit_grad.py:94)."""
    from kbench import percall as dropin
    from kbench.runtime import run_backward, run_forward

    static, theta, cw = _static("1", True, bicgstab_max_iter=1, bicgstab_tol=1e-30)
    fwd, bwd = (run_forward, run_backward) if path == "fused" else (dropin.run_forward, dropin.run_backward)
    _, saved = fwd(static, theta, cw)
    with pytest.raises(RuntimeError, match="BiCGSTAB"):
        bwd(static, theta, cw, saved)
        torch.cuda.synchronize()


def test_fused_backward_refuses_a_pibar_side_threshold():
    """The whole-pass backward alone refuses the option (``kbench.runtime.run_backward`` then takes the
    per-call path: tests/test_runtime_options_gpu.py)."""
    from kbench.runtime import run_backward_fused, run_forward

    static, theta, cw = _static("1", True, pibar_side_threshold=1e-3)
    _, saved = run_forward(static, theta, cw)
    with pytest.raises(NotImplementedError):
        run_backward_fused(static, theta, cw, saved)


def test_fused_backward_never_reuses_a_freed_forward():
    """A forward's stored split terms are reused only for that forward's own live Pi / Pibar tensors.

    The first forward's outputs are freed, then a per-call forward at another theta
    allocates buffers of the same shape (the allocator hands back the same blocks);
    the fused backward of that second point must equal the one after a fresh
    fused forward at the second theta.
    """
    from kbench import percall as dropin
    from kbench.runtime import fused_solver

    static, theta, cw = _static("1", True)
    solver = fused_solver(static)
    _, saved = solver.run_forward(theta, cw)
    ptr = saved["pi_wave"].data_ptr()
    del saved
    theta2 = theta + 0.25
    _, saved2 = dropin.run_forward(static, theta2, cw)
    print(f"  reused address: {saved2['pi_wave'].data_ptr() == ptr or saved2['pibar_wave'].data_ptr() == ptr}")
    gt_a, gc_a = solver.run_backward(theta2, cw, saved2)
    _, saved3 = solver.run_forward(theta2, cw)
    gt_b, gc_b = solver.run_backward(theta2, cw, saved3)
    torch.cuda.synchronize()
    rt, rc = kbtest.norm_rel_t(gt_a, gt_b), kbtest.norm_rel_t(gc_a, gc_b)
    print(f"  grad_theta rel={rt:.3e} grad_col rel={rc:.3e}")
    assert rt <= 1e-4 and rc <= 1e-4


def test_fused_column_weight_check_follows_each_tensor():
    """float64 column weights (converted by the driver) are classified afresh for every new tensor."""
    from kbench import percall as dropin
    from kbench.runtime import fused_solver

    static, theta, cw = _static("1", True)
    solver = fused_solver(static)
    S = int(cw.numel())
    flat64 = torch.zeros(S, dtype=torch.float64, device="cuda")
    l_flat, _ = solver.run_forward(theta, flat64)
    del flat64
    weighted = torch.as_tensor(np.random.default_rng(5).normal(size=S) * 0.5, dtype=torch.float64, device="cuda")
    l_w, _ = solver.run_forward(theta, weighted)
    l_ref, _ = dropin.run_forward(static, theta, weighted.float())
    torch.cuda.synchronize()
    rel = abs(float(l_w) - float(l_ref)) / abs(float(l_ref))
    print(f"  uniform loss={float(l_flat):.7g} weighted loss={float(l_w):.7g} per-call={float(l_ref):.7g}")
    assert float(l_w) != float(l_flat)
    assert rel <= 1e-5
