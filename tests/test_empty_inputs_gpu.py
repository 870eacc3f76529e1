"""Empty inputs through the drop-in wrappers: waves of no rows and waves without splits.

The reference's glue never issues these, but a caller of the wrappers may (an empty wave after a
layout filter, a leaf wave passed to the split wrappers).  Each wrapper returns its empty outputs
(``[0, S]`` rows, ``[0]`` masks) without a launch or an error, and leaves the caller's in-place
buffers bitwise unchanged.  The calls take the arguments of the per-call solve on the tiny
problem (``kbench.percall.SolvePlan``), cut to zero rows or zero splits.
"""

import pytest
import torch

import kbtest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup():
    from kbench.fused import problem_to_captured
    from kbench.percall import plan_of
    from kbench.runtime import make_static

    cap = problem_to_captured(kbtest.problem("tiny"))
    static = make_static(cap, "cuda")
    theta, cw = cap["inputs"]["theta"].cuda(), cap["inputs"]["col_weights"].cuda()
    plan = plan_of(static)
    _, sv = plan.forward(theta, cw)
    c = plan._row_consts(sv["E"], sv["Ebar"], sv["E_s1"], sv["E_s2"], sv["log_pS"], sv["log_pD"],
                         sv["max_coupling"])
    torch.cuda.synchronize()
    return plan, sv, c


def test_sweeps_and_leaf_initialisation_of_an_empty_wave(setup):
    from kbench.core.kernels.wave_step import compute_leaf_initial_wave_step, compute_wave_step

    print("[empty] sweep and leaf initialisation with W = 0", flush=True)
    plan, sv, c = setup
    h, S = plan.h, plan.S
    pi, pibar, rmax = sv["pi_wave"].clone(), sv["pibar_wave"].clone(), sv["pibar_row_max"].clone()
    before = [t.clone() for t in (pi, pibar, rmax)]
    consts = (c.mt, c.DL, c.Ebar, c.E, c.SL1, c.SL2, sv["col_log_probs"])
    compute_leaf_initial_wave_step(pibar, 0, 0, S, *consts, h["node_child1"], h["node_child2"],
                                   h["node_subtree_start"], h["node_subtree_end"], plan.leaf_idx, c.leaf,
                                   item_idx=plan.item_idx, use_col_weights=False)
    compute_wave_step(pi, pi, pibar, 0, 0, S, *consts, h["node_child1"], h["node_child2"], plan.topo[0],
                      plan.topo[3], None, leaf_state_idx=plan.leaf_idx, leaf_logp=c.leaf, item_idx=plan.item_idx,
                      pibar_row_max=rmax, store_final_pibar=True, has_leaf_term=True, use_col_weights=False)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip((pi, pibar, rmax), before))


def test_split_term_mask_and_adjoint_of_an_empty_wave(setup):
    from kbench.core.kernels.dts_fused import compute_dts_forward
    from kbench.core.kernels.wave_backward import active_mask_from_rhs_absmax_fused, wave_backward_uniform_fused

    print("[empty] split term, active mask and adjoint with W = 0", flush=True)
    plan, sv, c = setup
    h, S = plan.h, plan.S
    w = next(w for w in plan.waves if w.split)
    dts = compute_dts_forward(sv["pi_wave"], sv["pibar_wave"], w.sl, w.sr, h["node_child1"], h["node_child2"], 0,
                              w.reduce_idx, c.pD_par, c.pS_par, item_idx=plan.item_idx, log_split_probs=w.lsp,
                              item_offset=w.ws)
    assert tuple(dts.shape) == (0, S)
    rhs = torch.zeros((0, S), dtype=sv["pi_wave"].dtype, device="cuda")
    act = active_mask_from_rhs_absmax_fused(rhs, 1e-6)
    assert tuple(act.shape) == (0,) and act.dtype == torch.bool
    gcol = torch.zeros((S,), dtype=rhs.dtype, device="cuda")
    outs = wave_backward_uniform_fused(
        sv["pi_wave"], sv["pibar_wave"], 0, 0, S, None, rhs, c.mt, c.DL, c.Ebar, c.E, c.SL1, c.SL2,
        sv["col_log_probs"], h["node_child1"], h["node_child2"], None, neumann_terms=3,
        leaf_state_idx=plan.leaf_idx, leaf_logp=c.leaf, has_leaf_term=True, active_mask=act,
        node_parent=plan.topo[0], max_ancestor_depth=plan.topo[3], pibar_row_max=sv["pibar_row_max"],
        item_idx=plan.item_idx, item_indexed_consts=True, grad_col_log_probs=gcol, use_col_weights=False,
        **plan.levels)
    torch.cuda.synchronize()
    assert len(outs) == 7 and all(tuple(o.shape) == (0, S) for o in outs)
    assert not gcol.any()


def test_split_adjoint_and_pibar_vjp_without_splits(setup):
    from kbench.core.kernels.wave_backward import (dts_cross_backward_accum_fused,
                                                   uniform_cross_pibar_vjp_tree_from_ud_fused)

    print("[empty] split adjoint and Pibar VJP with N = 0 splits", flush=True)
    plan, sv, c = setup
    h, S = plan.h, plan.S
    w = next(w for w in plan.waves if w.split)
    pi, pibar = sv["pi_wave"], sv["pibar_wave"]
    v = torch.ones((w.W, S), dtype=pi.dtype, device="cuda")
    rhs = torch.zeros_like(pi)
    g_pD, g_pS, g_mt = torch.zeros_like(c.pD_par), torch.zeros_like(c.pS_par), torch.zeros_like(c.mt)
    gcol = torch.zeros((S,), dtype=pi.dtype, device="cuda")
    sl, sr, red = w.sl[:0], w.sr[:0], w.reduce_idx[:0]
    lsp = torch.zeros((0,), dtype=pi.dtype, device="cuda")
    ud, A, side_on, _, _ = dts_cross_backward_accum_fused(
        pi, pibar, v, w.ws, sl, sr, red, lsp, c.pD_par, c.pS_par, h["node_child1"], h["node_child2"], rhs, S,
        active_mask=None, merge_s_term=True, grad_log_pD=g_pD, grad_log_pS=g_pS, grad_mt=g_mt,
        accum_param_reductions=True, accum_mt_reduction=True, output_pibar_ud=True, output_pibar_side_active=True,
        mt_squeezed=c.mt, pibar_row_max=sv["pibar_row_max"], item_idx=plan.item_idx)
    assert tuple(ud.shape) == (0, S) and tuple(A.shape) == (0,) and tuple(side_on.shape) == (0,)
    out = uniform_cross_pibar_vjp_tree_from_ud_fused(
        pi, sv["col_log_probs"], ud, A, sl, sr, rhs, S, reduce_idx=red, pibar_row_max=sv["pibar_row_max"],
        skip_zero_sides=True, side_active=side_on, grad_col_log_probs=gcol, use_col_weights=False, **plan.levels)
    torch.cuda.synchronize()
    assert out is None
    assert not rhs.any() and not g_pD.any() and not g_pS.any() and not g_mt.any() and not gcol.any()
