"""Root-score VJP with an adjoint cache, and the Gauss-Newton HVP (reference newton/ggn.py:1-303).

``vjp_root_to_theta`` applies J^T = d(Pi_root)/dtheta^T to a root-score
cotangent by the backward's reverse wave sweep and E-adjoint solve (shared
with ``kbench.api._implicit_grad``); ``seed_root=None`` with
``drop_norm=False`` reproduces the loss gradient.  With ``cache`` it keeps
every wave's adjoint, split term and mask, the accumulated cotangents and the
E adjoint: the point cache of the exact HVP.  ``make_ggn_hvp`` returns
M v = J^T B J v with the root-softmax covariance B.
"""

from __future__ import annotations

import torch

from kbench.api._implicit_grad import _e_adjoint_and_theta_vjp, _reverse_wave_sweep, _safe_exp2_ratio
from kbench.core.inference.logspace import logsumexp2 as _logsumexp2

from newton.forward_tangent import jvp_root_scores

__all__ = ["vjp_root_to_theta", "make_ggn_hvp"]

_LN2 = 0.6931471805599453


@torch.no_grad()
def vjp_root_to_theta(static, sv, seed_root, theta, col_weights, *, drop_norm=True, neumann_terms=None,
                      use_pruning=None, bicgstab_tol=None, cache=None):
    """J^T seed_root -> (grad_theta, grad_col) (reference ggn.py:41-210), uniform column weights."""
    so = static.solver_options
    wl, sh = static.wave_layout, static.state_helpers
    neumann_terms = int(so.neumann_terms if neumann_terms is None else neumann_terms)
    use_pruning = bool(so.use_adjoint_pruning if use_pruning is None else use_pruning)
    Pi = sv["pi_wave"]
    root_ids = wl["root_row_ids"]
    if seed_root is None:
        root_Pi = Pi.index_select(0, root_ids)
        seed_root = -_safe_exp2_ratio(root_Pi, _logsumexp2(root_Pi, dim=-1, keepdim=True))
    acc = _reverse_wave_sweep(
        wl, sh, Pi_star_wave=Pi, Pibar_star_wave=sv["pibar_wave"], E_star=sv["E"], E_s1=sv["E_s1"], E_s2=sv["E_s2"],
        Ebar=sv["Ebar"], log_pS=sv["log_pS"], log_pD=sv["log_pD"], max_coupling_mat=sv["max_coupling"],
        col_log_probs=sv["col_log_probs"], use_col_weights=False, uniform_pibar_row_max=sv["pibar_row_max"],
        item_idx=static.rate_item_idx, seed_root=seed_root, neumann_terms=neumann_terms,
        self_loop_solver=so.self_loop_solver, adjoint_pruning_threshold=so.adjoint_pruning_threshold,
        use_adjoint_pruning=use_pruning, pibar_side_threshold=so.pibar_side_threshold, cache=cache)
    if cache is not None:
        cache["accum"] = dict(acc)
    return _e_adjoint_and_theta_vjp(
        sv["E"], sv["log_pS"], sv["log_pD"], sv["log_pL"], sv["max_coupling"], sv["col_log_probs"], False,
        acc["grad_E"], acc["grad_Ebar"], acc["grad_E_s1"], acc["grad_E_s2"], acc["grad_log_pD"], acc["grad_log_pS"],
        acc["grad_mc"], acc["grad_col"], int(root_ids.numel()), theta, col_weights, sh, statewise=static.statewise,
        itemwise=static.itemwise, bicgstab_max_iter=so.bicgstab_max_iter,
        bicgstab_tol=float(so.bicgstab_tol if bicgstab_tol is None else bicgstab_tol),
        bicgstab_breakdown_tol=so.bicgstab_breakdown_tol, drop_norm=drop_norm, cache=cache)


def make_ggn_hvp(static, theta, col_weights, sv, *, self_tol=None, self_max_iter=200, vjp_neumann_terms=None,
                 vjp_use_pruning=None, vjp_bicgstab_tol=None):
    """hvp(v) = J^T B J v with B_i = ln2 (diag q_i - q_i q_i^T) (reference ggn.py:272-303)."""
    root_ids = static.wave_layout["root_row_ids"]
    root_Pi = sv["pi_wave"].index_select(0, root_ids)
    q = _safe_exp2_ratio(root_Pi, _logsumexp2(root_Pi, dim=-1, keepdim=True))

    def hvp(v_vec):
        v = v_vec.reshape(theta.shape).to(theta.dtype)
        t = jvp_root_scores(static, theta, v, sv, self_tol=self_tol, self_max_iter=self_max_iter)
        u = _LN2 * q * (t - (q * t).sum(dim=-1, keepdim=True))
        gt, _ = vjp_root_to_theta(static, sv, u, theta, col_weights, drop_norm=True, neumann_terms=vjp_neumann_terms,
                                  use_pruning=vjp_use_pruning, bicgstab_tol=vjp_bicgstab_tol)
        return gt.reshape(-1)

    return hvp
