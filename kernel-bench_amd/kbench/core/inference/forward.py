"""Forward wave loop of the glue (reference kbench/core/inference/forward.py:8-117).

For every wave in order: the split term of the wave's rows
(``compute_dts_forward``), then ``pi_iters`` local iterations alternating
between the ``pi`` and ``pibar`` buffers -- iteration 0 is the leaf
initialisation on leaf waves and is skipped on split waves, iteration 1 of a
split wave reads the split term itself, the last iteration also stores Pibar
and the row max.  Same call sequence and arguments as the reference glue, on
the HIP-backed wrappers.
"""

from __future__ import annotations

import torch

from ..kernels.dts_fused import compute_dts_forward
from ..kernels.wave_step import compute_leaf_initial_wave_step, compute_wave_step
from ..parameters.extract_parameters import as_item_param, as_item_state


def pi_wave_forward(wave_layout, state_helpers, e, e_bar, e_s1, e_s2, log_p_s, log_p_d, max_coupling_mat,
                    col_log_probs, use_col_weights: bool = True, *, item_idx: torch.Tensor, pi_iters: int = 6,
                    pi_residual_out: torch.Tensor | None = None):
    """-> (root rows of Pi, Pi [C, S], Pibar [C, S], Pibar row max [C])."""
    pi_iters = int(pi_iters)
    if pi_iters < 2 or pi_iters % 2 != 0:
        raise ValueError("pi_iters must be an even integer at least 2")
    C = int(wave_layout["leaf_state_index"].numel())
    S = int(state_helpers["S"])
    dev, dt = e.device, e.dtype
    pi = torch.empty((C, S), dtype=dt, device=dev)
    pibar = torch.empty((C, S), dtype=dt, device=dev)
    row_max = torch.empty((C,), dtype=dt, device=dev)

    G = int(e.shape[0])
    E_i = as_item_state(e, S, G)
    Ebar_i = as_item_state(e_bar, S, G)
    Es1_i = as_item_state(e_s1, S, G)
    Es2_i = as_item_state(e_s2, S, G)
    mt_i = as_item_state(max_coupling_mat.squeeze(-1), S, G)
    pD_par = as_item_param(log_p_d, G, S)
    pS_par = as_item_param(log_p_s, G, S)
    pD_i = as_item_state(log_p_d, S, G)
    pS_i = as_item_state(log_p_s, S, G)
    DL = 1.0 + pD_i + E_i
    SL1 = pS_i + Es2_i
    SL2 = pS_i + Es1_i
    h = state_helpers
    leaf_idx = wave_layout["leaf_state_index"]

    for meta in wave_layout["wave_metas"]:
        ws, W = meta["start"], meta["W"]
        has_splits = "sl" in meta
        dts_r = None
        if has_splits:
            dts_r = compute_dts_forward(
                pi, pibar, meta["sl"], meta["sr"], h["node_child1"], h["node_child2"], W, meta["reduce_idx"],
                pD_par, pS_par, item_idx=item_idx, log_split_probs=meta.get("log_split_probs"),
                n_eq1=meta.get("n_eq1"), eq1_reduce_idx=meta.get("eq1_reduce_idx"), ge2_ptr=meta.get("ge2_ptr"),
                ge2_parent_ids=meta.get("ge2_parent_ids"), ge2_max_fanout=meta.get("ge2_max_fanout"),
                item_offset=ws)
        for it in range(pi_iters):
            src, dst = (pi, pibar) if it % 2 == 0 else (pibar, pi)
            if it == 0:
                if has_splits:
                    continue
                compute_leaf_initial_wave_step(
                    dst, ws, W, S, mt_i, DL, Ebar_i, E_i, SL1, SL2, col_log_probs, h["node_child1"],
                    h["node_child2"], h["node_subtree_start"], h["node_subtree_end"], leaf_idx, pS_i,
                    item_idx=item_idx, use_col_weights=use_col_weights)
                continue
            from_split = it == 1 and has_splits
            last = it == pi_iters - 1
            compute_wave_step(
                dts_r if from_split else src, dst, pibar, ws, W, S, mt_i, DL, Ebar_i, E_i, SL1, SL2, col_log_probs,
                h["node_child1"], h["node_child2"], h["node_parent"], int(h["max_ancestor_depth"]), dts_r,
                leaf_state_idx=leaf_idx, leaf_logp=pS_i, item_idx=item_idx, pibar_row_max=row_max,
                store_final_pibar=last, has_leaf_term=not has_splits, input_ws=0 if from_split else None,
                use_col_weights=use_col_weights, pi_residual_out=pi_residual_out if last else None)
    return pi[wave_layout["root_row_ids"]], pi, pibar, row_max


Pi_wave_forward = pi_wave_forward
