"""Split-term tangent on the HIP kernel (drop-in for the reference kbench/core/kernels/dts_tangent.py).

``compute_dts_tangent`` (reference dts_tangent.py:96-122, kernel 25-93): the
directional derivative of ``compute_dts_forward``,

    d_dts[w, s] = sum over the splits of row w of sum_k 2^(t_k - dts_r[w, s]) dt_k

for the five DTL split terms t_k (duplication, two transfers, two
speciations), 0 where dts_r is -inf.  The reference scatters every split into
its parent row with atomic adds; here one workgroup per row sums its splits
in increasing split order (the grouping of ``compute_dts_forward``), so the
result is bitwise reproducible.
"""

from __future__ import annotations

import torch

from . import _hip as H
from .dts_fused import split_groups

__all__ = ["compute_dts_tangent"]


def _rate(t, dt, dev):
    t = t if torch.is_tensor(t) else torch.as_tensor(t, device=dev)
    if t.ndim == 0:
        t = t.reshape(1, 1)
    return H.f(t, dt, dev)


def compute_dts_tangent(Pi, Pibar, dPi, dPibar, lefts, rights, node_child1, node_child2, W, reduce_idx, log_pD_vec,
                        log_pS_vec, dlog_pD_vec, dlog_pS_vec, dts_r, item_idx, *, log_split_probs=None, n_eq1=None,
                        eq1_reduce_idx=None, ge2_ptr=None, ge2_parent_ids=None, ge2_max_fanout=None, item_offset=0):
    """[W, S] tangent of the split term of every row of the wave (reference dts_tangent.py:96-122)."""
    W = int(W)
    H.require_device(Pi, "compute_dts_tangent")
    dt, dev = Pi.dtype, Pi.device
    S = int(Pi.shape[1])
    N = int(lefts.shape[0])
    out = torch.zeros((W, S), device=dev, dtype=dt)
    if N == 0 or W == 0:
        return out
    for name, t in (("Pi", Pi), ("Pibar", Pibar), ("dPi", dPi), ("dPibar", dPibar)):
        if not t.is_contiguous() or t.ndim != 2 or int(t.shape[1]) != S or t.dtype != dt:
            raise ValueError(f"{name} must be a contiguous [C, S] tensor of the Pi dtype")
    dts = dts_r.contiguous()
    if tuple(dts.shape) != (W, S) or dts.dtype != dt:
        raise ValueError("dts_r must be a [W, S] tensor of the Pi dtype")
    lsp = (torch.zeros((N,), device=dev, dtype=dt) if log_split_probs is None
           else H.f(log_split_probs.reshape(N), dt, dev))
    pD, pS = _rate(log_pD_vec, dt, dev), _rate(log_pS_vec, dt, dev)
    dpD, dpS = _rate(dlog_pD_vec, dt, dev), _rate(dlog_pS_vec, dt, dev)
    if not (pD.shape == pS.shape == dpD.shape == dpS.shape):
        raise ValueError("log_pD, log_pS and their tangents must have one layout")
    by_state = pD.ndim == 2 and int(pD.shape[1]) != 1
    row_stride = 0 if int(pD.shape[0]) == 1 else int(pD.stride(0))
    ptr, order = split_groups(reduce_idx.to(dev), W)
    sl, sr = H.i64(lefts, dev), H.i64(rights, dev)
    item = H.i64(item_idx, dev)
    c1, c2 = H.i64(node_child1, dev), H.i64(node_child2, dev)
    io = H.KbDtsTanIO(
        dtype=H.dtype_code(dt), S=S, W=W, param_by_state=int(by_state), N=N, item_offset=int(item_offset),
        param_row_stride=row_stride, node_child1=H.ptr(c1), node_child2=H.ptr(c2), Pi=H.ptr(Pi), Pibar=H.ptr(Pibar),
        dPi=H.ptr(dPi), dPibar=H.ptr(dPibar), sl=H.ptr(sl), sr=H.ptr(sr), log_split_probs=H.ptr(lsp),
        split_ptr=H.ptr(ptr), split_order=H.ptr(order), log_pD=H.ptr(pD), log_pS=H.ptr(pS), dlog_pD=H.ptr(dpD),
        dlog_pS=H.ptr(dpS), dts_r=H.ptr(dts), item_idx=H.ptr(item), out=H.ptr(out),
    )
    H.check(H.lib().kb_dts_tangent(io, H.stream(dev)))
    return out
