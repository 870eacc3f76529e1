"""Second-order contraction of the E-step backward on the HIP kernel (drop-in for the reference
kbench/core/kernels/e_step_so.py).

``e_step_backward_so`` (reference e_step_so.py:182-220): the E-step VJP maps
primals x = (E, E_new, E_s1, E_s2, Ebar, log_pS, log_pD, log_pL[, col]) and
cotangents g to parameter gradients, linearly in g; this returns its
derivative along dx at fixed g:

    dq_k = ln2 q_k (dt_k - dE_new),   q_k = g_new 2^(t_k - E_new)
    d_grad_E = 2 dq1 + dq2 + dq0 at the parent + dr (tot - excl) + r (dtot - dexcl)

with the Pibar part differentiated at a frozen row max.  One workgroup per
item row (float64 inside); d_grad_col is summed over item rows in a fixed
order instead of the reference's atomic adds.
"""

from __future__ import annotations

import torch

from ..parameters.extract_parameters import as_item_state
from . import _hip as H

__all__ = ["e_step_backward_so"]


def e_step_backward_so(E, E_new, E_s1, E_s2, Ebar, log_pS, log_pD, log_pL, col_log_probs, node_parent, node_child1,
                       node_child2, max_ancestor_depth, g_new, g_s1, g_s2, g_ebar, dE, dE_new, dE_s1, dE_s2, dEbar,
                       dlog_pS, dlog_pD, dlog_pL, dcol, *, use_col_weights=False):
    """(d_grad_E, d_grad_pS, d_grad_pD, d_grad_pL, d_grad_mc, d_grad_col) (reference e_step_so.py:182-220).

    g_s1 / g_s2 enter the VJP linearly and drop out of the contraction; they are accepted for
    the reference's signature.
    """
    H.require_device(E, "e_step_backward_so")
    dt, dev = E.dtype, E.device
    if E.ndim != 2:
        raise ValueError("E must be a [G, S] tensor")
    G, S = int(E.shape[0]), int(E.shape[1])
    mat = lambda x: H.f(as_item_state(x, S, G), dt, dev)
    xs = [mat(x) for x in (E, E_new, E_s1, E_s2, Ebar, log_pS, log_pD, log_pL, g_new, g_ebar, dE, dE_new, dE_s1,
                           dE_s2, dEbar, dlog_pS, dlog_pD, dlog_pL)]
    col = H.f(col_log_probs, dt, dev)
    dc = None if dcol is None else H.f(dcol, dt, dev)
    outs = [torch.empty((G, S), device=dev, dtype=dt) for _ in range(5)]
    col_rows = torch.empty((G, S), device=dev, dtype=dt)
    d_col = torch.zeros_like(col)
    if G == 0:
        return (*outs, d_col)
    tree = H.tree_from_parent(node_parent, node_child1, node_child2)
    (Ev, En, Es1, Es2, Eb, pS, pD, pL, gN, gB, dEv, dEn, dEs1, dEs2, dEb, dpS, dpD, dpL) = xs
    io = H.KbEStepSoIO(
        dtype=H.dtype_code(dt), G=G, use_col_weights=int(bool(use_col_weights)), E=H.ptr(Ev), E_new=H.ptr(En),
        E_s1=H.ptr(Es1), E_s2=H.ptr(Es2), Ebar=H.ptr(Eb), log_pS=H.ptr(pS), log_pD=H.ptr(pD), log_pL=H.ptr(pL),
        col_log_probs=H.ptr(col), g_new=H.ptr(gN), g_ebar=H.ptr(gB), dE=H.ptr(dEv), dE_new=H.ptr(dEn),
        dE_s1=H.ptr(dEs1), dE_s2=H.ptr(dEs2), dEbar=H.ptr(dEb), dlog_pS=H.ptr(dpS), dlog_pD=H.ptr(dpD),
        dlog_pL=H.ptr(dpL), dcol=H.ptr(dc), d_grad_E=H.ptr(outs[0]), d_grad_pS=H.ptr(outs[1]),
        d_grad_pD=H.ptr(outs[2]), d_grad_pL=H.ptr(outs[3]), d_grad_mc=H.ptr(outs[4]), col_rows=H.ptr(col_rows),
    )
    H.check(H.lib().kb_estep_backward_so(tree.handle, io, H.stream(dev)))
    H.sum_rows_into(d_col, col_rows)
    return (*outs, d_col)
