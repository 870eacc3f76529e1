"""Second-order contraction of the wave adjoint on the HIP kernel (drop-in for the reference
kbench/core/kernels/wave_so.py).

``wave_backward_so`` (reference wave_so.py:246-293): at the cached adjoint v
of a wave, the derivative along the primal tangents (dPi, dPibar, the
constant tangents, d_dts) of

* one transposed self-loop application A^T v (the seed correction of the
  tangent adjoint solve), and
* the parameter buckets aw0..aw4, aw345 = v w_L w~_k,

with the saved row max frozen.  One workgroup per row, float64 inside; the
subtree sums are a preorder prefix scan and the child-column scatter is a
gather from the parent column, so nothing is accumulated atomically.
"""

from __future__ import annotations

import torch

from . import _hip as H

__all__ = ["wave_backward_so"]


def wave_backward_so(Pi_star, dPi, Pibar_star, dPibar, v, ws, W, S, pibar_row_max, mc, DL, dDL, Ebar, dEbar, E, dE,
                     SL1, dSL1, SL2, dSL2, col_log_probs, node_child1, node_child2, node_parent, max_ancestor_depth,
                     dts_r=None, d_dts=None, *, leaf_state_idx, leaf_logp, dleaf_logp, item_idx, has_leaf_term=True,
                     use_col_weights=False, d_rhs=None):
    """(d_Av [W, S], d_aw0, d_aw1, d_aw2, d_aw345, d_aw3, d_aw4) (reference wave_so.py:246-293).

    With ``d_rhs`` [C, S] the wave's own rows of it are added to d_Av, which is then the seed
    of the tangent adjoint solve.
    """
    W, S, ws = int(W), int(S), int(ws)
    H.require_device(Pi_star, "wave_backward_so")
    dt, dev = Pi_star.dtype, Pi_star.device
    outs = tuple(torch.empty((W, S), device=dev, dtype=dt) for _ in range(7))
    if W <= 0:
        return outs
    for name, t in (("Pi_star", Pi_star), ("dPi", dPi), ("Pibar_star", Pibar_star), ("dPibar", dPibar)):
        if not t.is_contiguous() or t.ndim != 2 or int(t.shape[1]) != S or t.dtype != dt:
            raise ValueError(f"{name} must be a contiguous [C, S] tensor of the Pi dtype")
    vv = v.contiguous()
    if tuple(vv.shape) != (W, S) or vv.dtype != dt:
        raise ValueError("v must be a [W, S] tensor of the Pi dtype")
    if (dts_r is None) != (d_dts is None):
        raise ValueError("dts_r and d_dts must be given together")
    dts = dd = None
    if dts_r is not None:
        dts, dd = dts_r.contiguous(), d_dts.contiguous()
    cs = []
    for c in (DL, dDL, Ebar, dEbar, E, dE, SL1, dSL1, SL2, dSL2):
        t = H.f(c, dt, dev)
        cs.append(t.reshape(1, -1) if t.ndim == 1 else t)
    shape = tuple(cs[0].shape)
    cs = [c if tuple(c.shape) == shape else c.expand(*shape).contiguous() for c in cs]
    cstride = 0 if shape[0] == 1 else int(cs[0].stride(0))
    rhs = None
    if d_rhs is not None:
        rhs = d_rhs
        if not rhs.is_contiguous() or rhs.dtype != dt or int(rhs.shape[1]) != S:
            raise ValueError("d_rhs must be a contiguous [C, S] tensor of the Pi dtype")
    tree = H.tree_from_parent(node_parent, node_child1, node_child2)
    rm = H.f(pibar_row_max, dt, dev)
    col = H.f(col_log_probs, dt, dev)
    item, leaf = H.i64(item_idx, dev), H.i64(leaf_state_idx, dev)
    lp, dlp = H.f(leaf_logp, dt, dev), H.f(dleaf_logp, dt, dev)
    io = H.KbWaveSoIO(
        dtype=H.dtype_code(dt), S=S, W=W, use_col_weights=int(bool(use_col_weights)),
        use_leaf_index=int(bool(has_leaf_term)), ws=ws, const_stride=cstride, Pi=H.ptr(Pi_star), dPi=H.ptr(dPi),
        Pibar=H.ptr(Pibar_star), dPibar=H.ptr(dPibar), v=H.ptr(vv), pibar_row_max=H.ptr(rm), DL=H.ptr(cs[0]),
        dDL=H.ptr(cs[1]), Ebar=H.ptr(cs[2]), dEbar=H.ptr(cs[3]), E=H.ptr(cs[4]), dE=H.ptr(cs[5]), SL1=H.ptr(cs[6]),
        dSL1=H.ptr(cs[7]), SL2=H.ptr(cs[8]), dSL2=H.ptr(cs[9]), col_log_probs=H.ptr(col), item_idx=H.ptr(item),
        leaf_state=H.ptr(leaf), leaf_logp=H.ptr(lp), dleaf_logp=H.ptr(dlp), dts=H.ptr(dts), d_dts=H.ptr(dd),
        d_rhs=H.ptr(rhs), d_out=H.ptr(outs[0]), d_aw0=H.ptr(outs[1]), d_aw1=H.ptr(outs[2]), d_aw2=H.ptr(outs[3]),
        d_aw345=H.ptr(outs[4]), d_aw3=H.ptr(outs[5]), d_aw4=H.ptr(outs[6]),
    )
    H.check(H.lib().kb_wave_backward_so(tree.handle, io, H.stream(dev)))
    return outs
