"""Second-order contraction of the split-term backward on the HIP kernels (drop-in for the reference
kbench/core/kernels/dts_so.py).

``dts_backward_so`` (reference dts_so.py:233-303): at the cached adjoint v of
a wave, the derivative along (dPi, dPibar, dlog_pD, dlog_pS, dmt) of the
split-term backward -- the Pi cotangents scattered into the child rows, the
staged Pibar cotangents and the parameter cotangents -- and of the Pibar tree
VJP that routes the staged cotangents back into the child rows.  A split
kernel (one workgroup per split) and a tree kernel (one per split side)
write rows; they are added into ``d_rhs``, ``d_grad_col`` and the parameter
accumulators in a fixed order here, where the reference adds atomically.
"""

from __future__ import annotations

import torch

from . import _hip as H

__all__ = ["dts_backward_so"]


def _accum_param(acc, rows, parent_items):
    """acc += per-split rows [N, S] in each split's item row; acc is [G, S], [G, 1] or [G]."""
    G = int(acc.shape[0]) if acc.ndim >= 1 else 1
    S = int(rows.shape[1])
    if acc.ndim == 2 and int(acc.shape[1]) == S:
        if G == 1:
            H.sum_rows_into(acc[0], rows)
        else:
            H.scatter_add_rows(acc, rows, parent_items)
        return
    tmp = torch.zeros((G, S), device=rows.device, dtype=rows.dtype)
    if G == 1:
        H.sum_rows_into(tmp[0], rows)
    else:
        H.scatter_add_rows(tmp, rows, parent_items)
    acc += tmp.sum(dim=1).reshape(acc.shape)


def dts_backward_so(Pi, dPi, Pibar, dPibar, v, ws, meta, S, log_pD_param, log_pS_param, dlog_pD_param, dlog_pS_param,
                    mc_item, dmc_item, col_log_probs, node_child1, node_child2, node_parent, max_ancestor_depth,
                    pibar_row_max, item_idx, d_rhs, d_grad_pD, d_grad_pS, d_grad_mt, d_grad_col, *,
                    compact_level_ptr=None, compact_level_parents=None, compact_level_child1=None,
                    compact_level_child2=None, use_col_weights=False):
    """Accumulate the contraction into d_rhs [C, S], d_grad_pD / pS / mt and d_grad_col
    (reference dts_so.py:233-303).  The compact_level_* tables are accepted for the reference's
    signature; the subtree sums come from the species tree of node_parent / node_child*."""
    sl, sr = meta["sl"], meta["sr"]
    N = int(sl.numel())
    if N == 0:
        return
    S = int(S)
    H.require_device(Pi, "dts_backward_so")
    dt, dev = Pi.dtype, Pi.device
    for name, t in (("Pi", Pi), ("dPi", dPi), ("Pibar", Pibar), ("dPibar", dPibar), ("d_rhs", d_rhs)):
        if not t.is_contiguous() or t.ndim != 2 or int(t.shape[1]) != S or t.dtype != dt:
            raise ValueError(f"{name} must be a contiguous [C, S] tensor of the Pi dtype")
    lsp = meta.get("log_split_probs")
    lsp = torch.zeros((N,), device=dev, dtype=dt) if lsp is None else H.f(lsp.reshape(N), dt, dev)

    def rate(x):
        x = x if torch.is_tensor(x) else torch.as_tensor(x, device=dev)
        return H.f(x.reshape(1, 1) if x.ndim == 0 else x, dt, dev)

    pD, pS, dpD, dpS = rate(log_pD_param), rate(log_pS_param), rate(dlog_pD_param), rate(dlog_pS_param)
    if not (pD.shape == pS.shape == dpD.shape == dpS.shape):
        raise ValueError("log_pD, log_pS and their tangents must have one layout")
    by_state = pD.ndim == 2 and int(pD.shape[1]) != 1
    prow = 0 if int(pD.shape[0]) == 1 else int(pD.stride(0))
    mt, dmt = H.f(mc_item, dt, dev), H.f(dmc_item, dt, dev)
    mt = mt.reshape(1, -1) if mt.ndim == 1 else mt
    dmt = dmt.reshape(1, -1) if dmt.ndim == 1 else dmt
    if tuple(mt.shape) != tuple(dmt.shape) or int(mt.shape[1]) != S:
        raise ValueError("mc_item and dmc_item must be [G, S] tensors")
    mrow = 0 if int(mt.shape[0]) == 1 else int(mt.stride(0))
    vv = v.contiguous()
    sl64, sr64, red = H.i64(sl, dev), H.i64(sr, dev), H.i64(meta["reduce_idx"], dev)
    item = H.i64(item_idx, dev)
    tree = H.tree_from_parent(node_parent, node_child1, node_child2)
    rm, col = H.f(pibar_row_max, dt, dev), H.f(col_log_probs, dt, dev)
    c1, c2 = H.i64(node_child1, dev), H.i64(node_child2, dev)
    ud, dud, side, colrows = (torch.empty((2 * N, S), device=dev, dtype=dt) for _ in range(4))
    pDr, pSr, mtr = (torch.empty((N, S), device=dev, dtype=dt) for _ in range(3))
    start = int(meta["start"])
    io = H.KbDtsSoIO(
        dtype=H.dtype_code(dt), S=S, param_by_state=int(by_state), use_col_weights=int(bool(use_col_weights)), N=N,
        ws=int(ws), item_offset=start, param_row_stride=prow, mt_row_stride=mrow, Pi=H.ptr(Pi), dPi=H.ptr(dPi),
        Pibar=H.ptr(Pibar), dPibar=H.ptr(dPibar), v=H.ptr(vv), sl=H.ptr(sl64), sr=H.ptr(sr64), reduce_idx=H.ptr(red),
        log_split_probs=H.ptr(lsp), log_pD=H.ptr(pD), log_pS=H.ptr(pS), dlog_pD=H.ptr(dpD), dlog_pS=H.ptr(dpS),
        mt=H.ptr(mt), dmt=H.ptr(dmt), item_idx=H.ptr(item), pibar_row_max=H.ptr(rm), col_log_probs=H.ptr(col),
        node_child1=H.ptr(c1), node_child2=H.ptr(c2), ud=H.ptr(ud), dud=H.ptr(dud), side_rows=H.ptr(side),
        col_rows=H.ptr(colrows), pD_rows=H.ptr(pDr), pS_rows=H.ptr(pSr), mt_rows=H.ptr(mtr),
    )
    H.check(H.lib().kb_dts_backward_so(tree.handle, io, H.stream(dev)))
    H.scatter_add_rows(d_rhs, side, lambda: torch.cat((sl64, sr64)), static=(sl64, sr64))
    # accumulators that are one row of S states take their column sums in one launch
    blocks, rest = [], []
    for acc, rows in ((d_grad_col, colrows), (d_grad_pD, pDr), (d_grad_pS, pSr), (d_grad_mt, mtr)):
        row = acc.numel() == S and acc.is_contiguous() and acc.dtype == dt
        (blocks if row else rest).append((acc.view(-1) if row else acc, rows))
    if len({int(a.data_ptr()) for a, _ in blocks}) < len(blocks):
        rest, blocks = blocks + rest, []
    H.rows_sum_accum(blocks)
    parent_items = item[start + red]
    for acc, rows in rest:
        if acc is d_grad_col:
            H.sum_rows_into(d_grad_col, colrows)
        else:
            _accum_param(acc, rows, parent_items)
