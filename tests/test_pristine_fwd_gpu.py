"""Both HIP paths reproduce the reference's own forward on configs 1 and 2 (tests/golden/pristine_fwd_*.npz).

The fixtures are the reference's float32 outputs (frozen glue over its
pristine Triton kernels, kbench/runtime.py:63-75), written in the build
container by tests/golden/make_pristine_fwd.py.  The per-call drop-in path
(the reference's call sequence over kbench.core.kernels) and the native
whole-pass driver both run here at the fixture's pi_iters; the bar is the
forward's: loss relative 1e-5, arrays within 2e-4 absolute or 1e-5 relative
of the reference, with the same non-finite pattern.
"""

import numpy as np
import pytest
import torch

from test_pristine_fwd_cpu import ARRAYS, CASES, close_to_fixture, fixture, problem, rows_of

pytestmark = pytest.mark.gpu


def _inputs(case):
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    z = fixture(case)
    cap = problem_to_captured(problem(case))
    static = make_static(cap, "cuda")
    theta = torch.from_numpy(np.ascontiguousarray(z["theta"])).cuda()
    cw = cap["inputs"]["col_weights"].cuda()
    return z, static, theta, cw


def _check(tag, z, loss, saved):
    ref = float(z["loss"])
    rel = abs(float(loss) - ref) / abs(ref)
    print(f"  {tag}: loss got={float(loss):.9g} ref={ref:.9g} rel={rel:.3e}", flush=True)
    assert rel <= 1e-5
    for k in ARRAYS:
        got = rows_of(z, k, saved[k].detach().cpu().numpy().astype(np.float64))
        pattern, err = close_to_fixture(got, z[k])
        ma = float(np.abs(got[np.isfinite(z[k])] - z[k][np.isfinite(z[k])]).max())
        print(f"    {k}: pattern={pattern} max_abs={ma:.3e} rel1={err:.3e}")
        assert pattern and (ma <= 2e-4 or err <= 1e-5), k


@pytest.mark.parametrize("fuse", [False, True], ids=["one_launch_per_sweep", "fused_sweep_chains"])
@pytest.mark.parametrize("case", sorted(CASES))
def test_dropin_forward_matches_reference_fixture(case, fuse, monkeypatch):
    """The per-call path, with one launch per sweep and with each wave's sweep chain in one launch
    (KBENCH_FUSE_SWEEPS: float chains in linear space, reference forward.py:60-108)."""
    from kbench.core.kernels import wave_step
    from kbench.percall.solve import plan_of

    monkeypatch.setattr(wave_step, "FUSE_SWEEPS", fuse)
    print(f"[pristine-fwd dropin] case={case} fuse_sweeps={fuse}", flush=True)
    z, static, theta, cw = _inputs(case)
    loss, saved = plan_of(static).forward(theta, cw, pi_iters=int(z["pi_iters"]))
    torch.cuda.synchronize()
    _check("dropin", z, loss, saved)


@pytest.mark.parametrize("case", sorted(CASES))
def test_fused_forward_matches_reference_fixture(case):
    from kbench.fused import FusedSolver, solver_options_dict

    print(f"[pristine-fwd fused] case={case}", flush=True)
    z, static, theta, cw = _inputs(case)
    so = dict(solver_options_dict(static.solver_options), pi_iters=int(z["pi_iters"]))
    solver = FusedSolver(static, so)
    loss, saved = solver.run_forward(theta, cw)
    torch.cuda.synchronize()
    _check("fused", z, loss, saved)
