"""Exact Hessian-vector product of the loss, forward over reverse (reference newton/hvp_exact.py:1-409).

``build_point_cache`` runs the backward once at theta and keeps every wave's
adjoint v_k, split term and mask, the accumulated cotangents and the E
adjoint (theta is fixed across the CG iterations that use one point).
``make_exact_hvp(...)(u)`` then costs one tangent forward sweep
(``jvp_root_scores``) and one tangent reverse sweep with the same operators:
per wave, in reverse order, the second-order contraction at the cached
adjoint (``wave_backward_so``) seeds the tangent adjoint solve
(``wave_backward_uniform_fused`` with the cached mask); the tangent adjoint
goes through the split-term backward and its Pibar tree VJP, plus their own
contraction at the cached adjoint (``dts_backward_so``).  The E side adds
the E-step contractions (``e_step_backward_so``) and a BiCGSTAB tangent
E-adjoint solve; the parameter head adds the extraction's Hessian term by
autograd.  Same functions, arguments and call order as the reference.
"""

from __future__ import annotations

import os

import torch

from kbench.api._implicit_grad import _bicgstab, _safe_exp2_ratio
from kbench.core.inference.logspace import logsumexp2 as _logsumexp2
from kbench.core.kernels.dts_so import dts_backward_so
from kbench.core.kernels.dts_tangent import compute_dts_tangent
from kbench.core.kernels.e_step import e_step_triton_autograd
from kbench.core.kernels.e_step_so import e_step_backward_so
from kbench.core.kernels.wave_backward import (dts_cross_backward_accum_fused,
                                               uniform_cross_pibar_vjp_tree_from_ud_fused,
                                               wave_backward_uniform_fused)
from kbench.core.kernels.wave_so import wave_backward_so
from kbench.core.parameters.extract_parameters import as_item_param, as_item_state, extract_parameters_weighted_cols

from newton.forward_tangent import jvp_root_scores, wave_step_constants
from newton.ggn import vjp_root_to_theta

__all__ = ["build_point_cache", "make_exact_hvp"]

_LN2 = 0.6931471805599453


@torch.no_grad()
def build_point_cache(static, theta, col_weights, sv):
    """Backward once with the per-wave adjoints cached -> (grad_theta, grad_col, cache) (reference hvp_exact.py:37-44)."""
    cache: dict = {}
    gt, gc = vjp_root_to_theta(static, sv, None, theta, col_weights, drop_norm=False, cache=cache)
    return gt, gc, cache


def _scatter_accum(acc, items, contrib, G):
    contrib = contrib.to(acc.dtype)
    if G == 1:
        if acc.ndim == 1:
            acc[0] += contrib.sum()
        elif int(acc.shape[1]) == 1:
            acc[0, 0] += contrib.sum()
        else:
            acc[0] += contrib.sum(dim=0)
    elif acc.ndim == 1:
        acc.index_add_(0, items, contrib.sum(dim=1))
    elif int(acc.shape[1]) == 1:
        acc[:, 0].index_add_(0, items, contrib.sum(dim=1))
    else:
        acc.index_add_(0, items, contrib)


def _plus_folded(acc, x, G, S):
    """acc + x for an as_item_param-shaped accumulator and an item-state [G, S] term.

    With one parameter per item row (acc [G, 1]) the state axis of x is summed: the
    reference's broadcast add would count the accumulator once per state (it is only
    exercised there with per-state parameters, where both are [G, S]).
    """
    x = as_item_param(x, G, S)
    if int(acc.shape[-1]) == 1 and int(x.shape[-1]) != 1:
        x = x.sum(dim=-1, keepdim=True)
    return acc + x


def make_exact_hvp(static, theta, col_weights, sv, *, cache=None, debug_out=None, tangent_self_iters=None):
    """hvp(u_vec) -> H u (flat, theta's size) at theta (reference hvp_exact.py:54-383).

    ``tangent_self_iters``: fixed per-wave tangent sweeps of the forward tangent; default the
    ``NEWTON_TANGENT_SELF_ITERS`` environment variable, else ``solver_options.pi_iters``.
    """
    so = static.solver_options
    if tangent_self_iters is None:
        env = os.environ.get("NEWTON_TANGENT_SELF_ITERS")
        tangent_self_iters = int(env) if env else (int(so.pi_iters) if getattr(so, "pi_iters", None) else 16)
    sh, wl = static.state_helpers, static.wave_layout
    S = int(sh["S"])
    item_idx = static.rate_item_idx
    c1, c2, parent = sh["node_child1"], sh["node_child2"], sh["node_parent"]
    mad = int(sh["max_ancestor_depth"])
    leaf_state_idx = wl["leaf_state_index"]
    root_ids = wl["root_row_ids"]
    n_fam = int(root_ids.numel())
    dtype = sv["pi_wave"].dtype
    C = int(sv["pi_wave"].shape[0])
    E_star = sv["E"]
    G = int(E_star.shape[0])
    if cache is None:
        _, _, cache = build_point_cache(static, theta, col_weights, sv)
    acc = cache["accum"]
    wE = cache["e_side"]["wE"]
    cst = wave_step_constants(sv, S)
    prm = sv["pibar_row_max"]
    col = sv["col_log_probs"]
    item = lambda t: as_item_state(t, S, G)
    pS_m, pD_m, pL_m = item(sv["log_pS"]), item(sv["log_pD"]), item(sv["log_pL"])
    levels = dict(compact_level_ptr=sh["compact_level_ptr"], compact_level_parents=sh["compact_level_parents"],
                  compact_level_child1=sh["compact_level_child1"], compact_level_child2=sh["compact_level_child2"])

    # E-step graph at (E*, params): the transposed products that are linear in a cotangent
    E_req = E_star.detach().requires_grad_(True)
    with torch.enable_grad():
        E_new_g, E_s1_g, E_s2_g, Ebar_g = e_step_triton_autograd(
            E_req, sv["log_pS"], sv["log_pD"], sv["log_pL"], sv["max_coupling"], col, parent, c1, c2, mad,
            use_col_weights=False)

    def jt_E(g_new):
        with torch.enable_grad():
            (out,) = torch.autograd.grad(E_new_g, E_req, grad_outputs=g_new.contiguous(), retain_graph=True)
        return out

    def aux_T(g_s1, g_s2, g_ebar):
        with torch.enable_grad():
            (out,) = torch.autograd.grad((E_s1_g, E_s2_g, Ebar_g), E_req, grad_outputs=(g_s1, g_s2, g_ebar),
                                         retain_graph=True)
        return out

    norm = (1 - torch.exp2(E_star).mean(dim=-1, keepdim=True)).clamp_min(torch.finfo(dtype).tiny)
    fam_factor = 1.0 if G == n_fam else float(n_fam)

    def e_bwd_params(g_new, g_ebar):
        with torch.enable_grad():
            ins = [x.detach().requires_grad_(True)
                   for x in (pS_m, pD_m, pL_m, item(sv["max_coupling"].squeeze(-1)), col)]
            En, _, _, Eb = e_step_triton_autograd(E_star.detach(), *ins, parent, c1, c2, mad, use_col_weights=False)
            outs = torch.autograd.grad((En, Eb), ins, grad_outputs=(g_new, g_ebar), allow_unused=True)
        return tuple(torch.zeros_like(z) if o is None else o for o, z in zip(outs, (pS_m, pD_m, pL_m, pS_m, col)))

    # u-independent: primal parameter cotangents and the head's first-order graph
    base_p = e_bwd_params(wE, acc["grad_Ebar"])
    cot_pS = _plus_folded(acc["grad_log_pS"], base_p[0], G, S)
    cot_pD = _plus_folded(acc["grad_log_pD"], base_p[1], G, S)
    cot_pL = base_p[2]
    cot_mc = acc["grad_mc"] + base_p[3]
    cot_col = acc["grad_col"] + base_p[4]
    theta_req = theta.detach().requires_grad_(True)
    col_req = col_weights.detach().requires_grad_(True)
    with torch.enable_grad():
        pS_h, pD_h, pL_h, mt_h, col_h = extract_parameters_weighted_cols(
            theta_req, col_req, sh, statewise=static.statewise, itemwise=static.itemwise, uniform_fast=True)
        pS_hp, pD_hp = as_item_param(pS_h, G, S), as_item_param(pD_h, G, S)
        pL_hi = as_item_state(pL_h, S, G)
        mt_hi = as_item_state(mt_h.squeeze(-1) if mt_h.ndim == pS_h.ndim + 1 else mt_h, S, G)
        phi1 = ((pS_hp * cot_pS).sum() + (pD_hp * cot_pD).sum() + (pL_hi * cot_pL).sum() + (mt_hi * cot_mc).sum()
                + (col_h * cot_col).sum())
        (g1,) = torch.autograd.grad(phi1, theta_req, create_graph=True)

    def hvp(u_vec):
        u = u_vec.reshape(theta.shape).to(theta.dtype)
        with torch.no_grad():
            t_root, full = jvp_root_scores(static, theta, u, sv, return_full=True, keep_d_dts=False,
                                           self_iters=tangent_self_iters)
            dcst = full["dcst"]
            dPi, dPibar = full["dPi"], full["dPibar"]
            dpS_m, dpD_m, dpL_m = item(full["dlog_pS"]), item(full["dlog_pD"]), item(full["dlog_pL"])
            dE, dEbar_e, dE_s1, dE_s2 = full["dE"], full["dEbar"], full["dE_s1"], full["dE_s2"]

            root_Pi = sv["pi_wave"].index_select(0, root_ids)
            q = _safe_exp2_ratio(root_Pi, _logsumexp2(root_Pi, dim=-1, keepdim=True))
            d_seed = -_LN2 * q * (t_root - (q * t_root).sum(dim=-1, keepdim=True))
            d_rhs = torch.zeros((C, S), device=theta.device, dtype=dtype)
            d_rhs.index_copy_(0, root_ids, d_seed.to(dtype))
            d_gpD = torch.zeros_like(acc["grad_log_pD"])
            d_gpS = torch.zeros_like(acc["grad_log_pS"])
            d_gE, d_gEbar, d_gEs1, d_gEs2 = (torch.zeros_like(E_star) for _ in range(4))
            d_gmc = torch.zeros_like(acc["grad_mc"])
            d_gcol = torch.zeros((S,), device=theta.device, dtype=dtype)

            for wave in cache["waves"]:  # reverse wave order already
                ws, W, meta = wave["ws"], wave["W"], wave["meta"]
                v_k, dts_r, mask = wave["v"], wave["dts_r"], wave["active_mask"]
                has_leaf = wave["has_leaf_term"]
                d_dts = None
                if dts_r is not None:
                    d_dts = compute_dts_tangent(
                        sv["pi_wave"], sv["pibar_wave"], dPi, dPibar, meta["sl"], meta["sr"], c1, c2, W,
                        meta["reduce_idx"], cst["pd_param"], cst["ps_param"], dcst["dpd_param"], dcst["dps_param"],
                        dts_r, item_idx, log_split_probs=meta.get("log_split_probs"), item_offset=ws)
                d_Av, *c_aw = wave_backward_so(
                    sv["pi_wave"], dPi, sv["pibar_wave"], dPibar, v_k, ws, W, S, prm, cst["mc"], cst["dl"],
                    dcst["dDL"], cst["ebar"], dcst["dEbar"], cst["e"], dcst["dE"], cst["sl1"], dcst["dSL1"],
                    cst["sl2"], dcst["dSL2"], col, c1, c2, parent, mad, dts_r, d_dts, leaf_state_idx=leaf_state_idx,
                    leaf_logp=cst["leaf"], dleaf_logp=dcst["dleaf"], item_idx=item_idx, has_leaf_term=has_leaf,
                    use_col_weights=False, d_rhs=d_rhs)
                dv, *l_aw = wave_backward_uniform_fused(
                    sv["pi_wave"], sv["pibar_wave"], ws, W, S, dts_r, d_Av, cst["mc"], cst["dl"], cst["ebar"],
                    cst["e"], cst["sl1"], cst["sl2"], col, c1, c2, None, neumann_terms=int(so.neumann_terms),
                    leaf_state_idx=leaf_state_idx, leaf_logp=cst["leaf"], has_leaf_term=has_leaf, active_mask=mask,
                    node_parent=parent, max_ancestor_depth=mad, pibar_row_max=prm, item_idx=item_idx,
                    item_indexed_consts=True, grad_col_log_probs=d_gcol, use_col_weights=False,
                    self_loop_solver=so.self_loop_solver, return_last_increment=False, **levels)
                aw0, aw1, aw2, aw345, aw3, aw4 = (a + b for a, b in zip(c_aw, l_aw))
                if debug_out is not None:
                    debug_out.setdefault("wave_trace", []).append(
                        (ws, float(d_Av.abs().max()), float(dv.abs().max()), float(d_rhs.abs().max())))
                rows_i = item_idx[ws:ws + W]
                _scatter_accum(d_gpD, rows_i, aw0, G)
                _scatter_accum(d_gpS, rows_i, aw345, G)
                _scatter_accum(d_gE, rows_i, aw0 + aw2, G)
                _scatter_accum(d_gEbar, rows_i, aw1, G)
                _scatter_accum(d_gEs1, rows_i, aw4, G)
                _scatter_accum(d_gEs2, rows_i, aw3, G)
                _scatter_accum(d_gmc, rows_i, aw2, G)
                if dts_r is not None:
                    sl, sr = meta["sl"], meta["sr"]
                    gl, gr, side_act, _, _ = dts_cross_backward_accum_fused(
                        sv["pi_wave"], sv["pibar_wave"], dv, ws, sl, sr, meta["reduce_idx"],
                        meta.get("log_split_probs", sl.new_zeros((int(sl.numel()),), dtype=dtype)), cst["pd_param"],
                        cst["ps_param"], c1, c2, d_rhs, S, active_mask=mask, merge_s_term=True, grad_log_pD=d_gpD,
                        grad_log_pS=d_gpS, grad_mt=d_gmc, accum_param_reductions=True, accum_mt_reduction=True,
                        output_pibar_ud=True, output_pibar_side_active=True,
                        pibar_side_threshold=so.pibar_side_threshold, mt_squeezed=cst["mc"], pibar_row_max=prm,
                        grad_mt_two_stage=bool(d_gmc.ndim == 2 and int(d_gmc.shape[0]) == 1),
                        grad_mt_two_stage_tile_splits=128, skip_inactive_pibar_output_zero=True, item_idx=item_idx)
                    uniform_cross_pibar_vjp_tree_from_ud_fused(
                        sv["pi_wave"], col, gl, gr, sl, sr, d_rhs, S, active_mask=mask, reduce_idx=meta["reduce_idx"],
                        pibar_row_max=prm, skip_zero_sides=True, side_active=side_act, grad_col_log_probs=d_gcol,
                        use_col_weights=False, side_active_threshold=so.pibar_side_threshold, **levels)
                    dts_backward_so(
                        sv["pi_wave"], dPi, sv["pibar_wave"], dPibar, v_k, ws, meta, S, cst["pd_param"],
                        cst["ps_param"], dcst["dpd_param"], dcst["dps_param"], cst["mc"], dcst["dMC"], col, c1, c2,
                        parent, mad, prm, item_idx, d_rhs, d_gpD, d_gpS, d_gmc, d_gcol, use_col_weights=False,
                        **levels)

            # ---- E side
            del dPi, dPibar
            full.clear()
            x_args = (E_star.contiguous(), E_star.contiguous(), sv["E_s1"], sv["E_s2"], sv["Ebar"], pS_m, pD_m,
                      pL_m, col.contiguous(), parent, c1, c2, mad)
            dx = (dE, dE, dE_s1, dE_s2, dEbar_e, dpS_m, dpD_m, dpL_m, None)
            zero_g = torch.zeros_like(E_star)
            aux_lin = aux_T(d_gEs1, d_gEs2, d_gEbar)
            so_aux = e_step_backward_so(*x_args, zero_g, acc["grad_E_s1"], acc["grad_E_s2"], acc["grad_Ebar"], *dx,
                                        use_col_weights=False)
            e2E = torch.exp2(E_star)
            dnorm = -_LN2 * (e2E * dE).mean(dim=-1, keepdim=True)
            dg_norm = fam_factor * (-_LN2 * e2E * dE / (S * norm) + e2E * dnorm / (S * norm * norm))
            dq_E = d_gE + aux_lin + so_aux[0] + dg_norm
            so_w = e_step_backward_so(*x_args, wE, zero_g, zero_g, zero_g, *dx, use_col_weights=False)
            rhs_E = (dq_E + so_w[0]).reshape(-1)
            E_shape = E_star.shape

            def AG_flat(w_flat):
                return (w_flat.view(E_shape) - jt_E(w_flat.view(E_shape))).reshape(-1)

            dwE = _bicgstab(AG_flat, rhs_E, max_iter=so.bicgstab_max_iter, tol=float(so.bicgstab_tol),
                            breakdown_tol=so.bicgstab_breakdown_tol).view(E_shape)
            if debug_out is not None:
                debug_out.update(d_gE=d_gE.clone(), d_gpD=d_gpD.clone(), d_gpS=d_gpS.clone(), d_gmc=d_gmc.clone(),
                                 d_gEbar=d_gEbar.clone(), d_gEs1=d_gEs1.clone(), d_gEs2=d_gEs2.clone(),
                                 dq_E=dq_E.clone(), dwE=dwE.clone())
            lin_p = e_bwd_params(dwE, d_gEbar)
            so_p = e_step_backward_so(*x_args, wE, zero_g, zero_g, acc["grad_Ebar"], *dx, use_col_weights=False)
            d_cot_pS = _plus_folded(d_gpS, lin_p[0] + so_p[1], G, S)
            d_cot_pD = _plus_folded(d_gpD, lin_p[1] + so_p[2], G, S)
            d_cot_pL = lin_p[2] + so_p[3]
            d_cot_mc = d_gmc + lin_p[3] + so_p[4]
            d_cot_col = d_gcol + lin_p[4] + so_p[5]
        with torch.enable_grad():
            phi2 = ((pS_hp * d_cot_pS).sum() + (pD_hp * d_cot_pD).sum() + (pL_hi * d_cot_pL).sum()
                    + (mt_hi * d_cot_mc).sum() + (col_h * d_cot_col).sum())
            (out,) = torch.autograd.grad((g1 * u).sum() + phi2, theta_req, retain_graph=True)
        return out.reshape(-1)

    return hvp
