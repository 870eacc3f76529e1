"""Solve driver of the glue (reference kbench/core/inference/solver.py:1-142).

``solve_e_pi`` extracts the rate parameters, runs the E fixed point and the
forward wave loop; ``nll_from_root_rows`` is the loss.  Same functions,
arguments and returns as the reference, on the HIP-backed wrappers.
"""

from __future__ import annotations

import math

import torch

from kbench.core.inference.forward import pi_wave_forward
from kbench.core.inference.logspace import logsumexp2
from kbench.core.kernels.e_step import e_fixed_point_triton
from kbench.core.parameters.extract_parameters import (extract_parameters_uniform,
                                                       extract_parameters_weighted_cols)


def col_weights_are_uniform(col_weights: torch.Tensor) -> bool:
    """True when every column weight equals the first (one host read)."""
    flat = col_weights.detach().reshape(-1)
    return bool(torch.all(flat == flat[0]).item())


def solve_e_pi(static, theta: torch.Tensor, col_weights: torch.Tensor, *, warm_start_E=None, pi_iters=None,
               pi_residual_out=None):
    """-> (E, E_s1, E_s2, Ebar, root_rows, pi, pibar, pibar_row_max, log_pS, log_pD, log_pL, max_coupling,
    col_log_probs), the reference's return order (solver.py:16-96)."""
    so = static.solver_options
    so.validate()
    h = static.state_helpers
    S = int(h["S"])
    weighted = not col_weights_are_uniform(col_weights)
    if weighted:
        pS, pD, pL, mt, col = extract_parameters_weighted_cols(
            theta.detach(), col_weights.detach(), h, statewise=static.statewise, itemwise=static.itemwise)
    else:
        pS, pD, pL, mt = extract_parameters_uniform(
            theta.detach(), h["unnorm_row_max"].to(device=theta.device, dtype=theta.dtype),
            statewise=static.statewise, itemwise=static.itemwise)
        col = theta.new_full((S,), -math.log2(S))
    G = int(static.wave_layout["root_row_ids"].numel()) if static.itemwise else 1
    if warm_start_E is not None:
        E0 = warm_start_E.detach().to(theta).contiguous()
    else:
        E0 = theta.new_full((G, S), float(so.e_init))
    E, E_s1, E_s2, Ebar = e_fixed_point_triton(
        E0, log_pS=pS, log_pD=pD, log_pL=pL, max_coupling=mt, col_log_probs=col, use_col_weights=weighted,
        node_parent=h["node_parent"], node_child1=h["node_child1"], node_child2=h["node_child2"],
        max_ancestor_depth=int(h["max_ancestor_depth"]), max_iter=so.e_max_iter, tol=so.e_tol)
    root_rows, pi, pibar, row_max = pi_wave_forward(
        wave_layout=static.wave_layout, state_helpers=h, e=E, e_bar=Ebar, e_s1=E_s1, e_s2=E_s2, log_p_s=pS,
        log_p_d=pD, max_coupling_mat=mt, col_log_probs=col, use_col_weights=weighted, item_idx=static.rate_item_idx,
        pi_iters=so.pi_iters if pi_iters is None else int(pi_iters), pi_residual_out=pi_residual_out)
    return E, E_s1, E_s2, Ebar, root_rows, pi, pibar, row_max, pS, pD, pL, mt, col


def solve_forward_residual(static, theta, col_weights, *, pi_iters: int, warm_start_E=None):
    """Per-family max of the last sweep's max |Pi_new - Pi_old| (reference solver.py:99-128)."""
    C = int(static.wave_layout["leaf_state_index"].numel())
    resid = torch.zeros(C, device=theta.device, dtype=torch.float32)
    solve_e_pi(static, theta, col_weights, warm_start_E=warm_start_E, pi_iters=pi_iters, pi_residual_out=resid)
    fam = static.wave_layout["item_idx"].to(device=resid.device, dtype=torch.long)
    n_fam = int(static.item_index_tensor.numel())
    out = torch.zeros(n_fam, device=resid.device, dtype=torch.float32)
    out.scatter_reduce_(0, fam, resid, reduce="amax", include_self=True)
    return out


def nll_vector_from_root_rows(root_rows: torch.Tensor, E: torch.Tensor) -> torch.Tensor:
    """Per-family -(LSE(root) - log2 S - log2(1 - mean 2^E)) (reference solver.py:131-138)."""
    norm = (1 - torch.exp2(E).mean(dim=-1)).clamp_min(torch.finfo(E.dtype).tiny)
    return -(logsumexp2(root_rows, dim=-1) - math.log2(root_rows.shape[-1]) - torch.log2(norm))


def nll_from_root_rows(root_rows: torch.Tensor, E: torch.Tensor) -> torch.Tensor:
    return nll_vector_from_root_rows(root_rows, E).sum()
