"""Rate parameters from theta and column weights.

Same functions, argument meaning and shapes as the reference
kbench/core/parameters/extract_parameters.py (cited per function).  These run
as torch expressions so the glue can differentiate them with autograd (the
reference does the same); they are O(G * S) and not part of the hot path.
"""

from __future__ import annotations

import math

import torch

_LN2 = math.log(2.0)


def as_item_param(t, item_rows, S=None):
    """Parameter tensor -> [item_rows, 1] or [item_rows, S] (extract_parameters.py:8-15).

    0-d tensors broadcast to every item row; a 1-d tensor of length S with a
    single item row is a state vector, any other 1-d tensor holds one value per
    item row.
    """
    G = int(item_rows)
    if t.ndim == 0:
        return t.reshape(1, 1).expand(G, 1).contiguous()
    if t.ndim == 1:
        if S is not None and G == 1 and int(t.numel()) == int(S):
            return t.reshape(1, int(S)).contiguous()
        return t.reshape(G, 1).contiguous()
    return t.contiguous()


def as_item_state(t, S, item_rows):
    """Parameter tensor -> [item_rows, S] (extract_parameters.py:18-22)."""
    p = as_item_param(t, item_rows, S)
    if int(p.shape[1]) == int(S):
        return p.contiguous()
    return p.expand(int(item_rows), int(S)).contiguous()


def _log2_rates(theta):
    """log2 of softmax over [0, theta_D, theta_L, theta_T] in base-2 logits."""
    base = torch.cat((theta.new_zeros((*theta.shape[:-1], 1)), theta), dim=-1)
    return torch.log_softmax(base * _LN2, dim=-1) / _LN2


def extract_parameters_uniform(theta, unnorm_row_max, *, statewise=False, itemwise=False):
    """(log_pS, log_pD, log_pL, max_coupling) for uniform column weights (extract_parameters.py:25-34)."""
    r = _log2_rates(theta)
    log_pT = r[..., 3]
    if statewise and not itemwise:
        mt = log_pT + unnorm_row_max
    else:
        mt = log_pT.unsqueeze(-1) + unnorm_row_max
    return r[..., 0], r[..., 1], r[..., 2], mt


def col_log_probs_from_weights(col_weights: torch.Tensor) -> torch.Tensor:
    """log2 softmax of the column weights (extract_parameters.py:37-38)."""
    return torch.log_softmax(col_weights, dim=-1) / _LN2


def col_valid_log_normalizer(col_log_probs: torch.Tensor, node_parent: torch.Tensor,
                             max_ancestor_depth: int) -> torch.Tensor:
    """-log2(1 - sum of column probabilities over the ancestors-or-self of s).

    Reference extract_parameters.py:41-65: the ancestor chain is followed for
    max_ancestor_depth steps; columns whose ancestors hold all the mass get
    -inf.
    """
    S = int(col_log_probs.numel())
    dev = col_log_probs.device
    p = torch.exp2(col_log_probs)
    parent = node_parent.to(device=dev, dtype=torch.long)
    node = torch.arange(S, device=dev, dtype=torch.long)
    mass = torch.zeros((S,), device=dev, dtype=col_log_probs.dtype)
    zero = torch.zeros((), device=dev, dtype=col_log_probs.dtype)
    for _ in range(max(1, int(max_ancestor_depth))):
        ok = (node >= 0) & (node < S)
        idx = node.clamp(0, max(S - 1, 0))
        mass = mass + torch.where(ok, p.index_select(0, idx), zero)
        node = torch.where(ok, parent.index_select(0, idx), torch.full_like(node, -1))
    rest = 1.0 - mass
    tiny = torch.finfo(col_log_probs.dtype).tiny
    return torch.where(rest > 0.0, -torch.log2(rest.clamp_min(tiny)), col_log_probs.new_full((S,), float("-inf")))


def extract_parameters_weighted_cols(theta, col_weights, state_helpers, *, statewise=False, itemwise=False,
                                     uniform_fast=False):
    """(log_pS, log_pD, log_pL, max_coupling, col_log_probs) (extract_parameters.py:68-93).

    ``uniform_fast`` subtracts log2(S) from max_coupling, the form the glue's
    theta VJP uses when the column weights are uniform.
    """
    r = _log2_rates(theta)
    log_pT = r[..., 3]
    col = col_log_probs_from_weights(col_weights.to(device=theta.device, dtype=theta.dtype))
    norm = col_valid_log_normalizer(col, state_helpers["node_parent"], int(state_helpers["max_ancestor_depth"]))
    if statewise and not itemwise:
        mt = log_pT + norm
    else:
        mt = log_pT.unsqueeze(-1) + norm
    if uniform_fast:
        mt = mt - math.log2(int(state_helpers["S"]))
    return r[..., 0], r[..., 1], r[..., 2], mt, col
