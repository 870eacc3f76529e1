"""E-step tangent fixed point on the HIP kernel (drop-in for the reference kbench/core/kernels/e_step_tangent.py).

``e_tangent_fixed_point`` (reference e_step_tangent.py:174-208, kernel 27-125)
solves (I - J_E^EE) dE* = J_E^Ep dp at the frozen fixed point E* by
Richardson iteration, the linearisation of one E-step being

    dE_new = sum_k w_k dt_k,   w_k = 2^(t_k - E_new)
    dt = (dpS + dE[c1] + dE[c2], dpD + 2 dE, dE + dEbar, dpL)
    dEbar = (dRS - dAS) / (rowsum - ancestor sum) + dmax_coupling

and returns (dE*, dE_s1, dE_s2, dEbar) of the converged tangent.  The whole
iteration runs in one launch, one workgroup per item row, in float64 with the
primal weights kept in registers; the reference launches one step per
iteration and synchronises the host on the max difference.  The stopping test
(max|dE_new - dE| <= tol * max(1, max|dE_new|), at most ``max_iter`` steps) is
applied per item row; with one item row it is the reference's test.  Float32
rows too long for three float64 rows in LDS (S > 6741) run in float32
arithmetic, with ``tol`` floored at 8 float32 epsilons (9.5e-7): below that,
float32 rounding alone keeps the iterates apart.  ``n_iter_out`` (an int32 [G]
tensor, not in the reference's signature) receives each row's step count.
"""

from __future__ import annotations

import torch

from ..parameters.extract_parameters import as_item_state
from . import _hip as H

__all__ = ["e_tangent_fixed_point"]


def e_tangent_fixed_point(E_star, dlog_pS, dlog_pD, dlog_pL, dmax_coupling, log_pS, log_pD, log_pL, max_coupling,
                          col_log_probs, node_parent, node_child1, node_child2, max_ancestor_depth, *, max_iter=2000,
                          tol=1e-9, use_col_weights=True, dE0=None, n_iter_out=None):
    """(dE*, dE_s1, dE_s2, dEbar), each [G, S] (reference e_step_tangent.py:174-208)."""
    H.require_device(E_star, "e_tangent_fixed_point")
    dt, dev = E_star.dtype, E_star.device
    code = H.dtype_code(dt)
    E = E_star.contiguous()
    if E.ndim != 2:
        raise ValueError("E_star must be a [G, S] tensor")
    G, S = int(E.shape[0]), int(E.shape[1])
    mats = [H.f(as_item_state(p, S, G), dt, dev) for p in (log_pS, log_pD, log_pL, max_coupling)]
    dmats = [H.f(as_item_state(p, S, G), dt, dev) for p in (dlog_pS, dlog_pD, dlog_pL, dmax_coupling)]
    col = H.f(col_log_probs, dt, dev)
    d0 = None if dE0 is None else H.f(dE0, dt, dev)
    if d0 is not None and tuple(d0.shape) != (G, S):
        raise ValueError("dE0 must have the shape of E_star")
    if n_iter_out is not None and (n_iter_out.dtype != torch.int32 or n_iter_out.device != dev
                                   or not n_iter_out.is_contiguous() or tuple(n_iter_out.shape) != (G,)):
        raise ValueError("n_iter_out must be a contiguous int32 [G] tensor on the device of E_star")
    outs = [torch.empty((G, S), device=dev, dtype=dt) for _ in range(4)]
    if G == 0:
        return tuple(outs)
    tree = H.tree_from_parent(node_parent, node_child1, node_child2)
    io = H.KbETanIO(
        dtype=code, G=G, use_col_weights=int(bool(use_col_weights)), max_iter=max(1, int(max_iter)), tol=float(tol),
        E=H.ptr(E), log_pS=H.ptr(mats[0]), log_pD=H.ptr(mats[1]), log_pL=H.ptr(mats[2]),
        max_coupling=H.ptr(mats[3]), col_log_probs=H.ptr(col), dlog_pS=H.ptr(dmats[0]), dlog_pD=H.ptr(dmats[1]),
        dlog_pL=H.ptr(dmats[2]), dmax_coupling=H.ptr(dmats[3]), dE0=H.ptr(d0), dE=H.ptr(outs[0]),
        dE_s1=H.ptr(outs[1]), dE_s2=H.ptr(outs[2]), dEbar=H.ptr(outs[3]), n_iter=H.ptr(n_iter_out),
    )
    H.check(H.lib().kb_e_tangent_fixed_point(tree.handle, io, H.stream(dev)))
    return tuple(outs)
