"""Problems with one parameter row per item (``itemwise``): theta is [n_families, 3] and every clade
row reads its family's rates through ``rate_item_idx`` (reference kbench/runtime.py:47-60,
extract_parameters.py:25-34; the glue carries G = n_items rows of E and of the rate constants).

``kbench.runtime`` runs these on the per-call drivers.  Checks, on config 1's layout:

* forward against the oracle's forward, which covers item rows: loss rel 1e-5, E / E_s1 / E_s2 /
  Ebar rows [G, S] and the Pi / Pibar rows to float32 rounding;
* every family given the same rates: the loss equals the one-row problem's (the whole-pass driver,
  pinned against the oracle elsewhere) and the per-family gradients summed over the families equal
  its gradient (rel 1e-4), the column gradient too;
* the oracle's backward covers one item row only, so the item-row backward is also pinned by
  central differences: at a converged schedule (pi_iters 120, 200 Neumann terms, no pruning,
  BiCGSTAB tolerance 1e-13) the float64 per-call gradient along four seeded directions equals the
  central difference of the float64 per-call loss (step 1e-4) to rel 1e-6;
* the float32 runtime gradient equals the float64 per-call gradient at the default options
  (rel 1e-4).
"""

import dataclasses

import numpy as np
import pytest
import torch

import kbench_oracle as O
import kbtest

pytestmark = pytest.mark.gpu


def _problem(itemwise=True, **so):
    from kbench import synth

    cfg = dataclasses.replace(synth.config("1"), itemwise=itemwise)
    if so:
        cfg = dataclasses.replace(cfg, solver_options=dict(cfg.solver_options, **so))
    return synth.build_problem(cfg)


def _static(p):
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    cap = problem_to_captured(p)
    return make_static(cap, "cuda"), cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()


def test_itemwise_forward_matches_the_oracle():
    from kbench.runtime import run_forward

    print("[itemwise] forward vs oracle", flush=True)
    p = _problem()
    static, theta, cw = _static(p)
    assert static.itemwise and tuple(theta.shape) == (int(p["meta"]["n_items"]), 3)
    loss, saved = run_forward(static, theta, cw)
    torch.cuda.synchronize()
    prob = O.Problem.from_dict(p)
    th = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    ref_loss, ref = O.forward(prob, th, np.asarray(p["inputs"]["col_weights"], dtype=np.float64))
    rel = abs(float(loss) - ref_loss) / abs(ref_loss)
    print(f"  loss got={float(loss):.9g} ref={ref_loss:.9g} rel={rel:.3e}; E rows {tuple(saved['E'].shape)}")
    assert rel <= 1e-5
    assert tuple(saved["E"].shape) == tuple(np.asarray(ref["E"]).shape)
    for k in ("E", "E_s1", "E_s2", "Ebar"):
        ok, ma, _ = kbtest.compare_inf_safe(saved[k].cpu().numpy(), ref[k])
        print(f"  {k}: ok={ok} max_abs={ma:.3e}")
        assert ok and ma <= 1e-5
    for k in ("pi_wave", "pibar_wave", "pibar_row_max"):
        ok, ma, mr = kbtest.compare_inf_safe(saved[k].cpu().numpy(), ref[k])
        print(f"  {k}: ok={ok} max_abs={ma:.3e} max_rel={mr:.3e}")
        assert ok and (ma <= 2e-4 or mr <= 1e-5)


def test_equal_item_rates_give_the_one_row_solve():
    from kbench.runtime import run_backward, run_forward

    print("[itemwise] equal rates vs the one-row problem", flush=True)
    pg = _problem(itemwise=False)
    sg, theta_g, cw = _static(pg)
    pi = _problem()
    si, _, _ = _static(pi)
    n = int(pi["meta"]["n_items"])
    theta_i = theta_g.reshape(1, 3).repeat(n, 1).contiguous()
    lg, svg = run_forward(sg, theta_g, cw)
    gg, gcg = run_backward(sg, theta_g, cw, svg)
    li, svi = run_forward(si, theta_i, cw)
    gi, gci = run_backward(si, theta_i, cw, svi)
    torch.cuda.synchronize()
    rl = abs(float(li) - float(lg)) / abs(float(lg))
    rt = kbtest.norm_rel_t(gi.sum(dim=0), gg)
    rc = kbtest.norm_rel_t(gci, gcg)
    print(f"  loss rel={rl:.3e} sum_f grad_theta_f rel={rt:.3e} grad_col rel={rc:.3e}")
    assert rl <= 1e-5 and rt <= 1e-4 and rc <= 1e-4


def test_itemwise_gradient_against_central_differences():
    from kbench.percall.solve import SolvePlan

    print("[itemwise] float64 per-call gradient vs central differences", flush=True)
    p = _problem(pi_iters=120, neumann_terms=200, use_adjoint_pruning=False, adjoint_pruning_threshold=0.0,
                 bicgstab_tol=1e-13, e_tol=1e-14)
    static, theta, cw = _static(p)
    plan = SolvePlan(static)
    x0, cw64 = theta.double(), cw.double()
    _, sv = plan.forward(x0, cw64)
    g, _ = plan.backward(x0, cw64, sv)
    g = g.reshape(-1)
    rng = np.random.default_rng(5)
    h = 1e-4
    for i in range(4):
        u = torch.as_tensor(rng.normal(size=x0.numel()), dtype=torch.float64, device="cuda")
        u = (u / u.norm()).reshape(x0.shape)
        lp, _ = plan.forward(x0 + h * u, cw64)
        lm, _ = plan.forward(x0 - h * u, cw64)
        fd = (float(lp) - float(lm)) / (2.0 * h)
        an = float((g * u.reshape(-1)).sum())
        rel = abs(fd - an) / max(abs(an), 1e-12)
        print(f"  direction {i}: grad.u={an:.10e} central difference={fd:.10e} rel={rel:.3e}", flush=True)
        assert rel <= 1e-6


def test_itemwise_float32_runtime_gradient_matches_float64():
    from kbench.percall.solve import SolvePlan
    from kbench.runtime import needs_per_call_backward, run_backward, run_forward

    print("[itemwise] float32 runtime gradient vs float64 per-call", flush=True)
    p = _problem()
    static, theta, cw = _static(p)
    assert needs_per_call_backward(static)
    _, sv = run_forward(static, theta, cw)
    gt, gc = run_backward(static, theta, cw, sv)
    plan = SolvePlan(static)
    _, sv64 = plan.forward(theta.double(), cw.double())
    gt64, gc64 = plan.backward(theta.double(), cw.double(), sv64)
    torch.cuda.synchronize()
    rt, rc = kbtest.norm_rel_t(gt, gt64), kbtest.norm_rel_t(gc, gc64)
    print(f"  grad_theta rel={rt:.3e} grad_col rel={rc:.3e}")
    assert rt <= 1e-4 and rc <= 1e-4
