"""Split-reduction wrapper on the HIP kernel (drop-in for the reference kbench/core/kernels/dts_fused.py).

``compute_dts_forward`` (reference pristine dts_fused.py:171-231): for every
row w of the wave, the log-sum-exp over the row's splits of the five DTL split
terms.  The reference runs an eq1 kernel (rows with one split) and a two-stage
ge2 kernel (rows with several); here one workgroup per row reduces all of its
splits in increasing split order, which is the same sum.  The eq1 / ge2
metadata is accepted for signature compatibility; the grouping comes from
``reduce_idx``.
"""

from __future__ import annotations

import torch

from . import _hip as H

__all__ = ["compute_dts_forward"]


def split_groups(reduce_idx: torch.Tensor, W: int):
    """(ptr [W+1], order [N]) int32: the splits of row w are order[ptr[w]:ptr[w+1]], increasing.

    Cached on the identity of ``reduce_idx`` (static wave metadata)."""
    return H.static_cached(("split_groups", int(W), str(reduce_idx.device)), (reduce_idx,),
                           lambda: _split_groups(reduce_idx, W))


def _split_groups(reduce_idx: torch.Tensor, W: int):
    red = reduce_idx.to(dtype=torch.long).reshape(-1)
    counts = torch.bincount(red, minlength=int(W))[: int(W)]
    ptr = torch.zeros(int(W) + 1, device=red.device, dtype=torch.int32)
    ptr[1:] = torch.cumsum(counts, 0).to(torch.int32)
    order = torch.sort(red, stable=True).indices.to(torch.int32)
    return ptr, order


def compute_dts_forward(Pi, Pibar, lefts, rights, node_child1, node_child2, W, reduce_idx, log_pD_vec, log_pS_vec,
                        item_idx, *, log_split_probs=None, n_eq1=None, eq1_reduce_idx=None, ge2_ptr=None,
                        ge2_parent_ids=None, ge2_max_fanout=None, active_parent_rows=None, item_offset=0):
    """[W, S] split term of every row of the wave (-inf for rows without splits or inactive rows)."""
    W = int(W)
    H.require_device(Pi, "compute_dts_forward")
    dt, dev = Pi.dtype, Pi.device
    S = int(Pi.shape[1])
    N = int(lefts.shape[0])
    out = torch.empty((W, S), device=dev, dtype=dt)
    if W == 0:
        return out
    if not Pi.is_contiguous() or not Pibar.is_contiguous():
        raise ValueError("Pi and Pibar must be contiguous [C, S] tensors")
    lsp = (torch.zeros((N,), device=dev, dtype=dt) if log_split_probs is None
           else H.f(log_split_probs.reshape(N), dt, dev))
    pD = log_pD_vec if torch.is_tensor(log_pD_vec) else torch.as_tensor(log_pD_vec, device=dev)
    pS = log_pS_vec if torch.is_tensor(log_pS_vec) else torch.as_tensor(log_pS_vec, device=dev)
    if pD.ndim == 0:
        pD, pS = pD.reshape(1, 1), pS.reshape(1, 1)
    pD, pS = H.f(pD, dt, dev), H.f(pS, dt, dev)
    by_state = pD.ndim == 2 and int(pD.shape[1]) != 1
    row_stride = 0 if int(pD.shape[0]) == 1 else int(pD.stride(0))
    if N > 0:
        ptr, order = split_groups(reduce_idx.to(dev), W)
    else:
        ptr = torch.zeros(W + 1, device=dev, dtype=torch.int32)
        order = torch.zeros(1, device=dev, dtype=torch.int32)
    sl, sr = H.i64(lefts, dev), H.i64(rights, dev)
    item = H.i64(item_idx, dev)
    act = None
    if active_parent_rows is not None:
        act = active_parent_rows.to(device=dev, dtype=torch.bool).contiguous()
    c1, c2 = H.i64(node_child1, dev), H.i64(node_child2, dev)
    io = H.KbDtsIO(
        dtype=H.dtype_code(dt), S=S, W=W, param_by_state=int(by_state), N=N, item_offset=int(item_offset),
        param_row_stride=row_stride, node_child1=H.ptr(c1), node_child2=H.ptr(c2), Pi=H.ptr(Pi),
        Pibar=H.ptr(Pibar), sl=H.ptr(sl), sr=H.ptr(sr), log_split_probs=H.ptr(lsp), split_ptr=H.ptr(ptr),
        split_order=H.ptr(order), log_pD=H.ptr(pD), log_pS=H.ptr(pS), item_idx=H.ptr(item), active=H.ptr(act),
        out=H.ptr(out),
    )
    H.check(H.lib().kb_dts_forward(io, H.stream(dev)))
    return out
