"""Forward-mode tangent (JVP) of the root rows w.r.t. theta (reference newton/forward_tangent.py:1-209).

``jvp_root_scores(static, theta, v, sv)`` threads a tangent through the whole
forward solve in the reference's order:

1. the parameter tangent d(extract_parameters_uniform)/dtheta . v
   (``torch.func.jvp``, reference forward_tangent.py:29-41);
2. the E tangent fixed point (``e_tangent_fixed_point``);
3. per wave, in topological order, the split-term tangent
   (``compute_dts_forward`` + ``compute_dts_tangent``) and the self-loop
   tangent at the saved Pi* (``compute_wave_step_tangent_selfloop`` for a
   fixed count, or repeated ``compute_wave_step_tangent`` until the
   reference's convergence test holds).

Same function names, arguments and return values as the reference; the
kernels underneath are the HIP-backed wrappers of ``kbench.core.kernels``.
"""

from __future__ import annotations

import torch
from torch.func import jvp

from kbench.core.kernels.dts_fused import compute_dts_forward
from kbench.core.kernels.dts_tangent import compute_dts_tangent
from kbench.core.kernels.e_step_tangent import e_tangent_fixed_point
from kbench.core.kernels.wave_tangent import compute_wave_step_tangent, compute_wave_step_tangent_selfloop
from kbench.core.parameters.extract_parameters import as_item_param, as_item_state, extract_parameters_uniform

__all__ = ["param_jvp_uniform", "wave_step_constants", "jvp_root_scores"]


def param_jvp_uniform(static, theta, v):
    """(dlog_pS, dlog_pD, dlog_pL, dmax_coupling) along v (reference forward_tangent.py:29-41)."""
    urm = static.state_helpers["unnorm_row_max"].to(device=theta.device, dtype=theta.dtype)

    def f(th):
        return extract_parameters_uniform(th, urm, statewise=static.statewise, itemwise=static.itemwise)

    _, tangents = jvp(f, (theta,), (v,))
    return tangents


def wave_step_constants(sv, S):
    """Per-item constants of the sweep, as the forward builds them (reference forward_tangent.py:44-61)."""
    G = int(sv["E"].shape[0])
    e = as_item_state(sv["E"], S, G)
    ps = as_item_state(sv["log_pS"], S, G)
    pd = as_item_state(sv["log_pD"], S, G)
    return {
        "dl": 1.0 + pd + e, "ebar": as_item_state(sv["Ebar"], S, G), "e": e,
        "sl1": ps + as_item_state(sv["E_s2"], S, G), "sl2": ps + as_item_state(sv["E_s1"], S, G),
        "mc": as_item_state(sv["max_coupling"].squeeze(-1), S, G), "leaf": ps,
        "pd_param": as_item_param(sv["log_pD"], G, S), "ps_param": as_item_param(sv["log_pS"], G, S),
    }


def _default_tol(dtype):
    return 1e-12 if dtype == torch.float64 else 1e-6


def _wave_tangent_constants(static, theta, v, sv, S, e_tol, raw_out=None):
    """E and parameter tangents assembled into the sweep's tangent constants (reference forward_tangent.py:68-96)."""
    dpS, dpD, dpL, dmt = param_jvp_uniform(static, theta, v)
    sh = static.state_helpers
    dE, dE_s1, dE_s2, dEbar = e_tangent_fixed_point(
        sv["E"], dpS, dpD, dpL, dmt, sv["log_pS"], sv["log_pD"], sv["log_pL"], sv["max_coupling"],
        sv["col_log_probs"], sh["node_parent"], sh["node_child1"], sh["node_child2"], int(sh["max_ancestor_depth"]),
        max_iter=int(static.solver_options.e_max_iter), tol=e_tol, use_col_weights=False,
    )
    if raw_out is not None:
        raw_out.update(dlog_pS=dpS, dlog_pD=dpD, dlog_pL=dpL, dmax_coupling=dmt, dE=dE, dE_s1=dE_s1, dE_s2=dE_s2,
                       dEbar=dEbar)
    G = int(sv["E"].shape[0])
    de = as_item_state(dE, S, G)
    dps = as_item_state(dpS, S, G)
    dpd = as_item_state(dpD, S, G)
    return {
        "dDL": dpd + de, "dEbar": as_item_state(dEbar, S, G), "dE": de,
        "dSL1": dps + as_item_state(dE_s2, S, G), "dSL2": dps + as_item_state(dE_s1, S, G),
        "dMC": as_item_state(dmt.squeeze(-1), S, G), "dleaf": dps,
        "dpd_param": as_item_param(dpD, G, S), "dps_param": as_item_param(dpS, G, S),
    }


def jvp_root_scores(static, theta, v, sv, *, self_tol=None, self_max_iter=200, e_tol=None, self_iters=None,
                    return_full=False, keep_d_dts=True, fused_selfloop=True):
    """d(Pi_root)/dtheta . v -> [n_root_rows, S] (reference forward_tangent.py:99-209).

    ``self_iters`` runs a fixed number of tangent sweeps per wave (the
    primal's ``pi_iters`` truncation), in one launch when ``fused_selfloop``;
    ``self_iters=None`` sweeps until max|change| <= self_tol * max(1, max|dPi|)
    (at most ``self_max_iter``).  ``return_full`` also returns the dPi /
    dPibar buffers, per-wave d_dts, the tangent constants and the raw
    parameter / E tangents.
    """
    sh, wl = static.state_helpers, static.wave_layout
    S = int(sh["S"])
    if self_tol is None:
        self_tol = _default_tol(theta.dtype)
    if e_tol is None:
        e_tol = _default_tol(theta.dtype)
    item_idx = static.rate_item_idx
    leaf_state_idx = wl["leaf_state_index"]
    c1, c2, parent = sh["node_child1"], sh["node_child2"], sh["node_parent"]
    mad = int(sh["max_ancestor_depth"])

    base = wave_step_constants(sv, S)
    raw = {} if return_full else None
    dc = _wave_tangent_constants(static, theta, v, sv, S, e_tol, raw_out=raw)

    pi, pibar = sv["pi_wave"], sv["pibar_wave"]
    C = int(pi.shape[0])
    dpi = torch.zeros((C, S), device=pi.device, dtype=pi.dtype)
    dpibar = torch.zeros((C, S), device=pi.device, dtype=pi.dtype)
    d_dts_by_ws = {} if return_full else None
    consts = (base["mc"], dc["dMC"], base["dl"], dc["dDL"], base["ebar"], dc["dEbar"], base["e"], dc["dE"],
              base["sl1"], dc["dSL1"], base["sl2"], dc["dSL2"])
    common = dict(leaf_state_idx=leaf_state_idx, leaf_logp=base["leaf"], dleaf_logp=dc["dleaf"], item_idx=item_idx,
                  use_col_weights=False)

    def step(dts_r, d_dts, ws, W, has_leaf, store):
        compute_wave_step_tangent(pi, dpi, dpi, ws, W, S, *consts, sv["col_log_probs"], c1, c2, parent, mad, dts_r,
                                  d_dts, dPibar_out=(dpibar if store else None), has_leaf_term=has_leaf, **common)

    for meta in wl["wave_metas"]:
        ws, W = int(meta["start"]), int(meta["W"])
        has_splits = "sl" in meta
        if has_splits:
            lay = dict(log_split_probs=meta.get("log_split_probs"), n_eq1=meta.get("n_eq1"),
                       eq1_reduce_idx=meta.get("eq1_reduce_idx"), ge2_ptr=meta.get("ge2_ptr"),
                       ge2_parent_ids=meta.get("ge2_parent_ids"), ge2_max_fanout=meta.get("ge2_max_fanout"),
                       item_offset=ws)
            dts_r = compute_dts_forward(pi, pibar, meta["sl"], meta["sr"], c1, c2, W, meta["reduce_idx"],
                                        base["pd_param"], base["ps_param"], item_idx=item_idx, **lay)
            d_dts = compute_dts_tangent(pi, pibar, dpi, dpibar, meta["sl"], meta["sr"], c1, c2, W, meta["reduce_idx"],
                                        base["pd_param"], base["ps_param"], dc["dpd_param"], dc["dps_param"], dts_r,
                                        item_idx, **lay)
        else:
            dts_r = d_dts = None
        if return_full and d_dts is not None and keep_d_dts:
            d_dts_by_ws[ws] = d_dts
        has_leaf = not has_splits
        if self_iters is not None and fused_selfloop:
            compute_wave_step_tangent_selfloop(pi, dpi, ws, W, S, max(int(self_iters), 1), *consts,
                                               sv["col_log_probs"], c1, c2, parent, mad, dts_r, d_dts,
                                               dPibar_out=dpibar, has_leaf_term=has_leaf, **common)
        elif self_iters is not None:
            n_it = max(int(self_iters), 1)
            for _ in range(n_it - 1):
                step(dts_r, d_dts, ws, W, has_leaf, store=False)
            step(dts_r, d_dts, ws, W, has_leaf, store=True)
        else:
            prev = dpi.narrow(0, ws, W).clone()
            for _ in range(int(self_max_iter)):
                step(dts_r, d_dts, ws, W, has_leaf, store=False)
                cur = dpi.narrow(0, ws, W)
                diff = float((cur - prev).abs().max())
                scale = float(cur.abs().max())
                if diff <= self_tol * max(1.0, scale):
                    break
                prev = cur.clone()
            step(dts_r, d_dts, ws, W, has_leaf, store=True)

    roots = dpi.index_select(0, wl["root_row_ids"])
    if return_full:
        return roots, dict(dPi=dpi, dPibar=dpibar, d_dts=d_dts_by_ws, dcst=dc, **raw)
    return roots
