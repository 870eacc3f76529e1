"""GPU parity of the native whole-pass driver against the CPU oracle."""

import numpy as np
import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


def _run_fused_forward(name, statewise=None):
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    p = kbtest.problem(name, statewise)
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    solver = FusedSolver(static, static.solver_options)
    theta = cap["inputs"]["theta"].cuda()
    cw = cap["inputs"]["col_weights"].cuda()
    loss, saved = solver.run_forward(theta, cw)
    torch.cuda.synchronize()
    return solver, static, theta, cw, loss, saved


@pytest.mark.parametrize("name,statewise", [("tiny", None), ("1", None), ("1", True), ("2", None)])
def test_fused_forward_matches_oracle(name, statewise):
    print(f"[fused-forward] config={name} statewise={statewise}", flush=True)
    solver, static, theta, cw, loss, saved = _run_fused_forward(name, statewise)
    prob, ref_loss, ref = kbtest.oracle_forward(name, statewise)
    stats = solver.forward_stats()
    rel = abs(float(loss) - ref_loss) / abs(ref_loss)
    print(f"  loss got={float(loss):.9g} ref={ref_loss:.9g} rel={rel:.3e} nE={stats['n_e_iter']}/{ref['n_e_iter']}")
    assert rel <= 1e-5
    for k in ("E", "E_s1", "E_s2", "Ebar"):
        ok, ma, mr = kbtest.compare_inf_safe(saved[k].cpu().numpy(), ref[k])
        print(f"  {k}: ok={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
        assert ok and ma <= 1e-5
    for k in ("pi_wave", "pibar_wave", "pibar_row_max"):
        ok, ma, mr = kbtest.compare_inf_safe(saved[k].cpu().numpy(), ref[k])
        print(f"  {k}: ok={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
        assert ok and (ma <= 2e-4 or mr <= 1e-5)
