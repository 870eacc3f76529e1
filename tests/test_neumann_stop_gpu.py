"""The whole-pass backward's early stop of the Neumann series against the full series.

``FusedSolver(neumann_rtol=0)`` sums every ``neumann_terms`` term of every row,
as the reference's wave backward does (pristine wave_backward.py:1232-1269);
the default stops a row's series at its first term whose entries are all at
most 2^-24 of the row's largest right-hand-side entry.  Checked on the same
forward: the active masks are identical, the gradients agree to 1e-6
normwise (the dropped remainder is about 1e-7 of the adjoints, the size of
float32 rounding of the sums), every solved row of the full
series reports ``neumann_terms`` applications, and the early stop uses fewer
on average.  Rows of up to 2048 states run ``bwd_row_kernel`` (config 3 is the
bench's workload), longer ones ``bwd_row_large_kernel``.  Both settings are
also checked against the float64 oracle by the other whole-pass tests (the
default there).
"""

import numpy as np
import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


def _big_tree_problem(leaves, families):
    from kbench import synth

    cfg = synth.ProblemConfig(leaves, families, n_nni=1, family_leaves_median=21.0, family_leaves_sigma=0.6,
                              family_leaves_max=80, statewise=True, seed=17)
    return synth.build_problem(cfg)


@pytest.mark.parametrize("case", ["1", "2", "3", "big4095", "big8191"])
def test_early_stop_matches_the_full_series(case):
    from kbench.fused import DEFAULT_NEUMANN_RTOL, FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    print(f"[neumann-stop] case={case}", flush=True)
    if case.startswith("big"):
        p = _big_tree_problem(4096 if case == "big8191" else 2048, 3)
    else:
        p = kbtest.problem(case, True)
    cap = problem_to_captured(p)
    static = make_static(cap, "cuda")
    theta = cap["inputs"]["theta"].cuda()
    cw = cap["inputs"]["col_weights"].cuda()
    full = FusedSolver(static, static.solver_options, neumann_rtol=0.0)
    fast = FusedSolver(static, static.solver_options)
    assert fast.neumann_rtol == DEFAULT_NEUMANN_RTOL
    _, saved = full.run_forward(theta, cw)
    g_full = full.run_backward(theta, cw, saved, return_info=True)
    g_fast = fast.run_backward(theta, cw, saved, return_info=True)
    again = fast.run_backward(theta, cw, saved, return_info=True)
    torch.cuda.synchronize()
    n_terms = int(full.so["neumann_terms"])
    t_full = g_full[2]["neumann_terms"].cpu().numpy()
    t_fast = g_fast[2]["neumann_terms"].cpu().numpy()
    solved = t_full != 255
    rt = kbtest.norm_rel(g_fast[0].cpu().numpy(), g_full[0].cpu().numpy())
    rc = kbtest.norm_rel(g_fast[1].cpu().numpy(), g_full[1].cpu().numpy())
    print(f"  S={full.S} rows solved={int(solved.sum())}: terms full={n_terms}, early stop mean "
          f"{t_fast[solved].mean():.2f} max {int(t_fast[solved].max())}; grad_theta rel={rt:.2e} grad_col rel={rc:.2e}")
    assert np.array_equal(g_full[2]["active_mask"].cpu().numpy(), g_fast[2]["active_mask"].cpu().numpy())
    assert np.array_equal(solved, t_fast != 255)
    assert np.all(t_full[solved] == n_terms)
    assert np.all(t_fast[solved] <= n_terms) and np.all(t_fast[solved] >= 1)
    assert t_fast[solved].mean() < n_terms
    assert rt <= 1e-6 and rc <= 1e-6
    assert torch.equal(again[0], g_fast[0]) and torch.equal(again[1], g_fast[1])


def test_neumann_rtol_from_the_environment(monkeypatch):
    from kbench.fused import FusedSolver, problem_to_captured
    from kbench.runtime import make_static

    print("[neumann-stop] KB_NEUMANN_RTOL", flush=True)
    cap = problem_to_captured(kbtest.problem("tiny", None))
    static = make_static(cap, "cuda")
    monkeypatch.setenv("KB_NEUMANN_RTOL", "0")
    assert FusedSolver(static, static.solver_options).neumann_rtol == 0.0
    with pytest.raises(ValueError):
        FusedSolver(static, static.solver_options, neumann_rtol=1.5)
