"""``kbench.runtime`` with the backward options the whole-pass driver does not implement, and the
version counters of the in-place wrapper outputs.

* ``self_loop_solver="gmres"`` and ``pibar_side_threshold > 0`` (reference kbench/runtime.py:77-115,
  pristine wave_backward.py:574-653, 1777-1884, 2263-2266): ``run_backward`` runs the per-call
  drivers and matches the oracle's backward with the same option (gradients rel 1e-4);
  ``run_backward_fused`` refuses them.  The side threshold is set at the median of the oracle's
  side bounds, so about half the split sides drop out of the Pibar VJP.
* A per-call ``compute_wave_step`` that writes into a whole-pass forward's saved ``pi_wave``
  bumps its version, so the whole-pass backward recomputes the split terms instead of reusing
  the ones its forward stored: its gradients equal those of the same backward on a fresh copy
  of the modified tensors, bitwise.
"""

import dataclasses

import numpy as np
import pytest
import torch

import kbench_oracle as O
import kbtest

pytestmark = pytest.mark.gpu


def _static(name, statewise, **opts):
    from kbench.fused import problem_to_captured
    from kbench.runtime import make_static

    cap = problem_to_captured(kbtest.problem(name, statewise))
    cap["meta"]["solver_options"] = dict(cap["meta"]["solver_options"], **opts)
    return make_static(cap, "cuda"), cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()


def _oracle_backward(name, statewise, **opts):
    p = kbtest.problem(name, statewise)
    prob, _, saved = kbtest.oracle_forward(name, statewise)
    prob = dataclasses.replace(prob, so=dict(prob.so, **opts))
    theta = np.asarray(p["inputs"]["theta"], dtype=np.float32).astype(np.float64)
    cw = np.asarray(p["inputs"]["col_weights"], dtype=np.float64)
    gt, gc, _info, extra = O.backward(prob, theta, cw, saved, collect=True)
    return gt, gc, extra


def _side_threshold(name, statewise):
    _, _, extra = _oracle_backward(name, statewise)
    b = np.concatenate(extra["side_bounds"])
    return float(np.median(b[b > 0]))


@pytest.mark.parametrize("name,statewise,option", [("1", True, "gmres"), ("1", None, "gmres"),
                                                   ("1", True, "side"), ("2", None, "side")])
def test_runtime_backward_takes_the_per_call_path_for_its_options(name, statewise, option):
    from kbench.runtime import needs_per_call_backward, run_backward, run_backward_fused, run_forward

    # GMRES with three iterations (at 16 it matches the 16-term Neumann series to 1e-11 here)
    base = {"neumann_terms": 3} if option == "gmres" else {}
    opts = (dict(base, self_loop_solver="gmres") if option == "gmres"
            else {"pibar_side_threshold": _side_threshold(name, statewise)})
    print(f"[runtime option] config={name} statewise={statewise} {opts}", flush=True)
    static, theta, cw = _static(name, statewise, **opts)
    assert needs_per_call_backward(static)
    _, saved = run_forward(static, theta, cw)
    gt, gc = run_backward(static, theta, cw, saved)
    torch.cuda.synchronize()
    ref_gt, ref_gc, extra = _oracle_backward(name, statewise, **opts)
    base_gt, _, _ = _oracle_backward(name, statewise, **base)
    rt, rc = kbtest.norm_rel(gt.cpu().numpy(), ref_gt), kbtest.norm_rel(gc.cpu().numpy(), ref_gc)
    shift = kbtest.norm_rel(ref_gt, base_gt)
    print(f"  grad_theta rel={rt:.3e} grad_col rel={rc:.3e} (the option moves grad_theta by {shift:.3e})")
    assert rt <= 1e-4 and rc <= 1e-4
    assert shift > 1e-4  # the option changes the gradient, and the runtime follows it
    with pytest.raises(NotImplementedError):
        run_backward_fused(static, theta, cw, saved)


def test_a_per_call_write_into_saved_pi_is_seen_by_the_fused_backward():
    from kbench.core.kernels.wave_step import compute_wave_step
    from kbench.percall.solve import plan_of
    from kbench.runtime import fused_solver

    print("[version counters] per-call sweep into a fused forward's saved rows", flush=True)
    static, theta, cw = _static("1", True)
    solver = fused_solver(static)
    # the constants of another point (computed first: the backward below may reuse only the split
    # terms of the solver's most recent forward)
    _, saved2 = solver.run_forward(theta + 0.3, cw)
    _, saved = solver.run_forward(theta, cw)
    ref_gt, ref_gc = solver.run_backward(theta, cw, saved)  # the stored split terms reused
    # one sweep of the first leaf wave, with the other point's constants, into the saved rows
    plan = plan_of(static)
    c = plan._row_consts(saved2["E"], saved2["Ebar"], saved2["E_s1"], saved2["E_s2"], saved2["log_pS"],
                         saved2["log_pD"], saved2["max_coupling"])
    w = next(w for w in plan.waves if not w.split)
    h = plan.h
    v0, vb0 = saved["pi_wave"]._version, saved["pibar_wave"]._version
    compute_wave_step(saved["pi_wave"], saved["pi_wave"], saved["pibar_wave"], w.ws, w.W, plan.S, c.mt, c.DL,
                      c.Ebar, c.E, c.SL1, c.SL2, saved2["col_log_probs"], h["node_child1"], h["node_child2"],
                      plan.topo[0], plan.topo[3], None, leaf_state_idx=plan.leaf_idx, leaf_logp=c.leaf,
                      item_idx=plan.item_idx, pibar_row_max=saved["pibar_row_max"], store_final_pibar=True,
                      has_leaf_term=True, use_col_weights=False)
    assert saved["pi_wave"]._version > v0 and saved["pibar_wave"]._version > vb0
    gt_a, gc_a = solver.run_backward(theta, cw, saved)
    fresh = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in saved.items()}
    gt_b, gc_b = solver.run_backward(theta, cw, fresh)
    torch.cuda.synchronize()
    moved = kbtest.norm_rel_t(gt_a, ref_gt)
    print(f"  the write moves grad_theta by rel {moved:.3e}; modified vs fresh copy: "
          f"equal={torch.equal(gt_a, gt_b) and torch.equal(gc_a, gc_b)}")
    assert moved > 1e-6
    assert torch.equal(gt_a, gt_b) and torch.equal(gc_a, gc_b)
