"""Implicit-gradient glue of the backward (reference kbench/api/_implicit_grad.py:1-475).

``implicit_grad_loglik_vjp_wave`` walks the waves in reverse: active mask of
the wave's accumulated adjoint rows, split term with inactive parents masked,
self-loop adjoint and parameter contributions, split adjoint into the
children and the Pibar VJP of the staged cotangents.  The E-adjoint is then
solved with BiCGSTAB on (I - J_E^T) and pulled back to theta and the column
weights with autograd through the E-step and the parameter extraction.  Same
functions, arguments and call sequence as the reference glue, on the
HIP-backed wrappers.
"""

from __future__ import annotations

import torch

from kbench.core.inference.logspace import logsumexp2 as _logsumexp2
from kbench.core.kernels.dts_fused import compute_dts_forward
from kbench.core.kernels.e_step import e_step_triton_autograd
from kbench.core.kernels.wave_backward import (active_mask_from_rhs_absmax_fused, dts_cross_backward_accum_fused,
                                               uniform_cross_pibar_vjp_tree_from_ud_fused,
                                               wave_backward_uniform_fused)
from kbench.core.parameters.extract_parameters import (as_item_param, as_item_state,
                                                       extract_parameters_weighted_cols)

_NEG_INF = float("-inf")


def _safe_exp2_ratio(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """2^(a - b), 0 where a is -inf."""
    dead = a == _NEG_INF
    return torch.where(dead, torch.zeros_like(a), torch.exp2(torch.where(dead, 0.0, a) - torch.where(dead, 0.0, b)))


def _norm(x) -> float:
    return float(torch.linalg.vector_norm(x).detach().cpu())


@torch.no_grad()
def _bicgstab(Av, b: torch.Tensor, *, max_iter: int = 500, tol: float = 1e-7, breakdown_tol: float = 1e-30):
    """BiCGSTAB for A x = b with the reference's stopping and breakdown rules (_implicit_grad.py:27-94).

    Relative residuals are measured against max(||b||, 1); a breakdown
    (|rho|, |<r_hat, v>|, <t, t> or |omega| at most breakdown_tol) or running
    out of iterations raises RuntimeError.
    """
    max_iter, tol, breakdown_tol = int(max_iter), float(tol), float(breakdown_tol)
    if max_iter < 1:
        raise ValueError("max_iter must be at least 1")
    if tol <= 0.0:
        raise ValueError("tol must be positive")
    if breakdown_tol <= 0.0:
        raise ValueError("breakdown_tol must be positive")
    x = torch.zeros_like(b)
    r = b - Av(x)
    scale = max(_norm(b), 1.0)
    rel = _norm(r) / scale
    if rel <= tol:
        return x
    r0 = r.clone()
    one = torch.ones((), dtype=b.dtype, device=b.device)
    rho_prev, alpha, omega = one.clone(), one.clone(), one.clone()
    v = torch.zeros_like(b)
    p = torch.zeros_like(b)
    k = 0
    for k in range(1, max_iter + 1):
        rho = torch.dot(r0, r)
        if float(rho.abs().cpu()) <= breakdown_tol:
            break
        p = r + (rho / rho_prev) * (alpha / omega) * (p - omega * v)
        v = Av(p)
        den = torch.dot(r0, v)
        if float(den.abs().cpu()) <= breakdown_tol:
            break
        alpha = rho / den
        s = r - alpha * v
        if _norm(s) / scale <= tol:
            return x + alpha * p
        t = Av(s)
        tt = torch.dot(t, t)
        if float(tt.abs().cpu()) <= breakdown_tol:
            break
        omega = torch.dot(t, s) / tt
        x = x + alpha * p + omega * s
        r = s - omega * t
        rel = _norm(r) / scale
        if rel <= tol:
            return x
        if float(omega.abs().cpu()) <= breakdown_tol:
            break
        rho_prev = rho
    raise RuntimeError(f"E-adjoint BiCGSTAB solve failed after {k} iterations (relative residual {rel:.3e})")


@torch.no_grad()
def implicit_grad_loglik_vjp_wave(wave_layout, state_helpers, *, Pi_star_wave, Pibar_star_wave, E_star, E_s1, E_s2,
                                  Ebar, log_pS, log_pD, log_pL, max_coupling_mat, col_log_probs, use_col_weights,
                                  theta, col_weights, uniform_pibar_row_max, item_idx, statewise=False,
                                  itemwise=False, neumann_terms=3, self_loop_solver="neumann",
                                  bicgstab_max_iter=500, bicgstab_tol=1e-7, bicgstab_breakdown_tol=1e-30,
                                  adjoint_pruning_threshold=1e-6, use_adjoint_pruning=True,
                                  pibar_side_threshold=0.0, collect_backward_relres=False):
    """(grad_theta, grad_col) of the summed loss (reference _implicit_grad.py:97-369)."""
    neumann_terms = int(neumann_terms)
    if neumann_terms < 0:
        raise ValueError("neumann_terms must be non-negative")
    self_loop_solver = str(self_loop_solver).strip().lower()
    if self_loop_solver not in ("neumann", "gmres"):
        raise ValueError("self_loop_solver must be one of: neumann, gmres")
    thr = float(adjoint_pruning_threshold)
    if thr < 0.0:
        raise ValueError("adjoint_pruning_threshold must be non-negative")
    side_thr = float(pibar_side_threshold)
    if side_thr < 0.0:
        raise ValueError("pibar_side_threshold must be non-negative")

    roots = wave_layout["root_row_ids"]
    root_pi = Pi_star_wave.index_select(0, roots)
    seed = -_safe_exp2_ratio(root_pi, _logsumexp2(root_pi, dim=-1, keepdim=True))
    acc = _reverse_wave_sweep(
        wave_layout, state_helpers, Pi_star_wave=Pi_star_wave, Pibar_star_wave=Pibar_star_wave, E_star=E_star,
        E_s1=E_s1, E_s2=E_s2, Ebar=Ebar, log_pS=log_pS, log_pD=log_pD, max_coupling_mat=max_coupling_mat,
        col_log_probs=col_log_probs, use_col_weights=use_col_weights, uniform_pibar_row_max=uniform_pibar_row_max,
        item_idx=item_idx, seed_root=seed, neumann_terms=neumann_terms, self_loop_solver=self_loop_solver,
        adjoint_pruning_threshold=thr, use_adjoint_pruning=use_adjoint_pruning, pibar_side_threshold=side_thr,
        collect_backward_relres=collect_backward_relres)
    if collect_backward_relres:
        return acc
    return _e_adjoint_and_theta_vjp(
        E_star, log_pS, log_pD, log_pL, max_coupling_mat, col_log_probs, use_col_weights, acc["grad_E"],
        acc["grad_Ebar"], acc["grad_E_s1"], acc["grad_E_s2"], acc["grad_log_pD"], acc["grad_log_pS"], acc["grad_mc"],
        acc["grad_col"], int(roots.numel()), theta, col_weights, state_helpers, statewise=statewise,
        itemwise=itemwise, bicgstab_max_iter=bicgstab_max_iter, bicgstab_tol=bicgstab_tol,
        bicgstab_breakdown_tol=bicgstab_breakdown_tol)


@torch.no_grad()
def _reverse_wave_sweep(wave_layout, state_helpers, *, Pi_star_wave, Pibar_star_wave, E_star, E_s1, E_s2, Ebar,
                        log_pS, log_pD, max_coupling_mat, col_log_probs, use_col_weights, uniform_pibar_row_max,
                        item_idx, seed_root, neumann_terms, self_loop_solver, adjoint_pruning_threshold,
                        use_adjoint_pruning, pibar_side_threshold, collect_backward_relres=False, cache=None):
    """Reverse wave sweep of the adjoint from a root-row seed (reference _implicit_grad.py:199-353).

    Returns the accumulated cotangents (grad_E, grad_Ebar, grad_E_s1, grad_E_s2, grad_log_pD,
    grad_log_pS, grad_mc, grad_col).  With ``cache`` (a dict) every wave's adjoint (inactive
    rows zeroed), split term and active mask are appended to ``cache["waves"]`` in sweep order
    (the point cache of newton/ggn.py:41-210).
    """
    thr, side_thr = float(adjoint_pruning_threshold), float(pibar_side_threshold)
    C, S = Pi_star_wave.shape
    dev, dt = Pi_star_wave.device, Pi_star_wave.dtype
    G = int(E_star.shape[0])
    E_i, Ebar_i, pS_i, pD_i, mt_i = (as_item_state(x, S, G) for x in (E_star, Ebar, log_pS, log_pD, max_coupling_mat))
    pD_par, pS_par = (as_item_param(x, G, S) for x in (log_pD, log_pS))
    DL_i = 1.0 + pD_i + E_i
    SL1_i = pS_i + as_item_state(E_s2, S, G)
    SL2_i = pS_i + as_item_state(E_s1, S, G)

    rhs_all = torch.zeros(C, S, device=dev, dtype=dt)
    g_pD, g_pS = torch.zeros_like(pD_par), torch.zeros_like(pS_par)
    g_mt = torch.zeros_like(mt_i)
    g_col = torch.zeros((S,), device=dev, dtype=dt)
    g_E, g_Ebar, g_Es1, g_Es2 = (torch.zeros_like(x) for x in (E_star, Ebar, E_star, E_star))

    roots = wave_layout["root_row_ids"]
    rhs_all.index_copy_(0, roots, seed_root.to(dt))

    def add_rows(acc, items, contrib):
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

    h = state_helpers
    levels = (h["compact_level_ptr"], h["compact_level_parents"], h["compact_level_child1"],
              h["compact_level_child2"])
    leaf_idx = wave_layout["leaf_state_index"].to(device=dev, dtype=torch.int32).contiguous()

    relres_fam = vk_fam = row_item = None
    if collect_backward_relres:
        row_item = wave_layout["item_idx"].to(device=dev, dtype=torch.long)
        n_fam = int(row_item.max().item()) + 1 if row_item.numel() else 0
        relres_fam = torch.zeros(n_fam, device=dev, dtype=torch.float32)
        vk_fam = torch.zeros(n_fam, device=dev, dtype=torch.float32)

    for meta in reversed(wave_layout["wave_metas"]):
        ws, W = int(meta["start"]), int(meta["W"])
        rhs_k = rhs_all[ws: ws + W]
        active = active_mask_from_rhs_absmax_fused(rhs_k, thr, use_pruning=bool(use_adjoint_pruning)).contiguous()
        has_splits = bool(meta.get("has_splits", "sl" in meta))
        has_leaf = int(meta.get("phase", 1 if not has_splits else 2)) == 1
        dts_r = None
        if has_splits:
            dts_r = compute_dts_forward(
                Pi_star_wave.detach(), Pibar_star_wave.detach(), meta["sl"], meta["sr"], h["node_child1"],
                h["node_child2"], W, meta["reduce_idx"], pD_par, pS_par, item_idx=item_idx,
                log_split_probs=meta.get("log_split_probs"), n_eq1=meta.get("n_eq1"),
                eq1_reduce_idx=meta.get("eq1_reduce_idx"), ge2_ptr=meta.get("ge2_ptr"),
                ge2_parent_ids=meta.get("ge2_parent_ids"), ge2_max_fanout=meta.get("ge2_max_fanout"),
                active_parent_rows=active, item_offset=ws)
        out = wave_backward_uniform_fused(
            Pi_star_wave, Pibar_star_wave, ws, W, S, dts_r, rhs_k, mt_i, DL_i, Ebar_i, E_i, SL1_i, SL2_i,
            col_log_probs, h["node_child1"], h["node_child2"], None, neumann_terms=neumann_terms,
            leaf_state_idx=leaf_idx, leaf_logp=pS_i, has_leaf_term=has_leaf, active_mask=active,
            node_parent=h["node_parent"], max_ancestor_depth=int(h["max_ancestor_depth"]),
            pibar_row_max=uniform_pibar_row_max, item_idx=item_idx, item_indexed_consts=True,
            compact_level_ptr=levels[0], compact_level_parents=levels[1], compact_level_child1=levels[2],
            compact_level_child2=levels[3], grad_col_log_probs=g_col, use_col_weights=use_col_weights,
            self_loop_solver=self_loop_solver, return_last_increment=collect_backward_relres)
        if collect_backward_relres:
            v_k, aw0, aw1, aw2, aw345, aw3, aw4, last = out
            items_w = row_item[ws: ws + W]
            on = active.reshape(active.shape[0], -1).ne(0).any(dim=1)
            vk_norm = torch.where(on, v_k.float().norm(dim=1), torch.zeros(W, device=dev, dtype=torch.float32))
            vk_fam.scatter_reduce_(0, items_w, vk_norm, reduce="amax", include_self=True)
            if last is not None:
                relres_fam.scatter_reduce_(0, items_w, last.float(), reduce="amax", include_self=True)
        else:
            v_k, aw0, aw1, aw2, aw345, aw3, aw4 = out
        if cache is not None:
            on = active.reshape(W, -1).ne(0).any(dim=1)
            cache.setdefault("waves", []).append(dict(
                ws=ws, W=W, v=torch.where(on.unsqueeze(1), v_k, torch.zeros_like(v_k)), dts_r=dts_r,
                active_mask=active, has_splits=has_splits, has_leaf_term=has_leaf, meta=meta))
        items = item_idx[ws: ws + W]
        add_rows(g_pD, items, aw0)
        add_rows(g_pS, items, aw345)
        add_rows(g_E, items, aw0 + aw2)
        add_rows(g_Ebar, items, aw1)
        add_rows(g_Es1, items, aw4)
        add_rows(g_Es2, items, aw3)
        add_rows(g_mt, items, aw2)
        if has_splits:
            sl, sr = meta["sl"], meta["sr"]
            ud, A, side_active, _, _ = dts_cross_backward_accum_fused(
                Pi_star_wave, Pibar_star_wave, v_k, ws, sl, sr, meta["reduce_idx"],
                meta.get("log_split_probs", sl.new_zeros((int(sl.numel()),), dtype=dt)), pD_par, pS_par,
                h["node_child1"], h["node_child2"], rhs_all, S, active_mask=active, merge_s_term=True,
                grad_log_pD=g_pD, grad_log_pS=g_pS, grad_mt=g_mt, accum_param_reductions=True,
                accum_mt_reduction=True, output_pibar_ud=True, output_pibar_side_active=True,
                pibar_side_threshold=side_thr, mt_squeezed=mt_i, pibar_row_max=uniform_pibar_row_max,
                grad_mt_two_stage=bool(g_mt.ndim == 2 and int(g_mt.shape[0]) == 1),
                grad_mt_two_stage_tile_splits=128, skip_inactive_pibar_output_zero=True, item_idx=item_idx)
            uniform_cross_pibar_vjp_tree_from_ud_fused(
                Pi_star_wave, col_log_probs, ud, A, sl, sr, rhs_all, S, active_mask=active,
                reduce_idx=meta["reduce_idx"], pibar_row_max=uniform_pibar_row_max, skip_zero_sides=True,
                side_active=side_active, compact_level_ptr=levels[0], compact_level_parents=levels[1],
                compact_level_child1=levels[2], compact_level_child2=levels[3], grad_col_log_probs=g_col,
                use_col_weights=use_col_weights, side_active_threshold=side_thr)
    if collect_backward_relres:
        return relres_fam, vk_fam
    return dict(grad_E=g_E, grad_Ebar=g_Ebar, grad_E_s1=g_Es1, grad_E_s2=g_Es2, grad_log_pD=g_pD, grad_log_pS=g_pS,
                grad_mc=g_mt, grad_col=g_col)


def _e_adjoint_and_theta_vjp(E_star, log_pS, log_pD, log_pL, max_coupling_mat, col_log_probs, use_col_weights,
                             grad_E, grad_Ebar, grad_E_s1, grad_E_s2, grad_log_pD, grad_log_pS,
                             grad_max_coupling_mat, grad_col_log_probs, n_fam, theta, col_weights, state_helpers, *,
                             statewise, itemwise, bicgstab_max_iter=500, bicgstab_tol=1e-7,
                             bicgstab_breakdown_tol=1e-30, drop_norm=False, cache=None):
    """E adjoint by BiCGSTAB on (I - J_E^T) w = q_E, then the theta / column VJP (reference _implicit_grad.py:372-475).

    ``drop_norm`` leaves out the loss's explicit log2(1 - mean 2^E) term (a root-score
    cotangent instead of the loss, newton/ggn.py:213-244); ``cache`` receives the E-side
    adjoint (``cache["e_side"]``: q_E, wE, aux_to_e).
    """
    topo = (state_helpers["node_parent"], state_helpers["node_child1"], state_helpers["node_child2"],
            int(state_helpers["max_ancestor_depth"]))
    E_req = E_star.detach().requires_grad_(True)
    with torch.enable_grad():
        E_new, Es1_new, Es2_new, Ebar_new = e_step_triton_autograd(
            E_req, log_pS, log_pD, log_pL, max_coupling_mat, col_log_probs, *topo, use_col_weights=use_col_weights)
        outs, gouts = (Es1_new, Es2_new, Ebar_new), (grad_E_s1, grad_E_s2, grad_Ebar)
        if not drop_norm:
            norm = (1 - torch.exp2(E_req).mean(dim=-1)).clamp_min(torch.finfo(E_req.dtype).tiny)
            denom = torch.log2(norm)
            direct = denom.sum() if E_req.shape[0] == n_fam else (n_fam * denom).sum()
            outs, gouts = (direct, *outs), (torch.ones_like(direct), *gouts)
        (aux,) = torch.autograd.grad(outs, E_req, grad_outputs=gouts, retain_graph=True)
    q_E = grad_E + aux
    q = q_E.reshape(-1)
    shape = E_star.shape

    def apply(w_flat):
        w = w_flat.view(shape).contiguous()
        with torch.enable_grad():
            (jt,) = torch.autograd.grad(E_new, E_req, grad_outputs=w.clone(), retain_graph=True)
        return (w - jt).reshape(-1)

    wE = _bicgstab(apply, q, max_iter=bicgstab_max_iter, tol=bicgstab_tol,
                   breakdown_tol=bicgstab_breakdown_tol).view(shape)
    if cache is not None:
        cache["e_side"] = dict(q_E=q_E, wE=wE, aux_to_e=aux)

    theta_req = theta.detach().requires_grad_(True)
    col_req = col_weights.detach().requires_grad_(True)
    with torch.enable_grad():
        pS_r, pD_r, pL_r, mt_r, col_r = extract_parameters_weighted_cols(
            theta_req, col_req, state_helpers, statewise=statewise, itemwise=itemwise,
            uniform_fast=not use_col_weights)
        S = int(state_helpers["S"])
        G = int(E_star.shape[0])
        loss_p = ((as_item_param(pS_r, G, S) * grad_log_pS).sum() + (as_item_param(pD_r, G, S) * grad_log_pD).sum()
                  + (mt_r * grad_max_coupling_mat).sum() + (col_r * grad_col_log_probs).sum())
        E_p, _, _, Ebar_p = e_step_triton_autograd(E_star.detach(), pS_r, pD_r, pL_r, mt_r, col_r, *topo,
                                                   use_col_weights=use_col_weights)
        grad_theta, grad_col = torch.autograd.grad((loss_p, Ebar_p, E_p), (theta_req, col_req),
                                                   grad_outputs=(torch.ones_like(loss_p), grad_Ebar, wE))
    return grad_theta, grad_col
