"""Wave-sweep tangents on the HIP kernel (drop-in for the reference kbench/core/kernels/wave_tangent.py).

* ``compute_wave_step_tangent`` -- one tangent application of the sweep
  (reference wave_tangent.py:392-431, kernel 35-177);
* ``compute_wave_step_tangent_selfloop`` -- ``n_iters`` in-place tangent
  sweeps of a wave in one launch (reference wave_tangent.py:346-389, kernel
  181-343).

Per row, at the frozen primal row Pi: the sweep is Pi_new = LSE(t0..t5[, dts])
with t0 = DL + Pi, t1 = Pi + Ebar, t2 = pibar + E, t3 = SL1 + Pi[c1],
t4 = SL2 + Pi[c2], t5 = the leaf term, so

    dPi_new = sum_k 2^(t_k - Pi_new) dt_k,
    dpibar  = (dRS - dAS) / (rowsum - ancestor sum) + dMC.

The primal weights are computed once per launch and kept in registers; the
tangent row lives in LDS, in float64, and the ancestor sums of r * dPi are one
Euler-tour prefix scan instead of the reference's bounded ancestor chase.
"""

from __future__ import annotations

import torch

from . import _hip as H

__all__ = ["compute_wave_step_tangent", "compute_wave_step_tangent_selfloop"]


def _const_stride(c) -> int:
    return 0 if int(c.shape[0]) == 1 else int(c.stride(0))


def _launch(Pi_in, dPi_in, dPi_out, ws, W, S, n_iters, pi_ws, consts, col_log_probs, node_child1, node_child2,
            node_parent, DTS_reduced, dDTS, leaf_state_idx, leaf_logp, dleaf_logp, item_idx, dPibar_out,
            has_leaf_term, use_col_weights, what):
    W, S, ws = int(W), int(S), int(ws)
    if W <= 0:
        return
    H.require_device(Pi_in, what)
    dt, dev = Pi_in.dtype, Pi_in.device
    named = [("Pi_in", Pi_in), ("dPi_in", dPi_in), ("dPi_out", dPi_out)]
    if dPibar_out is not None:
        named.append(("dPibar_out", dPibar_out))
    for name, t in named:
        if not t.is_contiguous() or t.ndim != 2 or int(t.shape[1]) != S:
            raise ValueError(f"{name} must be a contiguous [*, S] tensor")
        if t.dtype != dt:
            raise RuntimeError(f"{name} has dtype {t.dtype}, expected {dt}")
    has_splits = DTS_reduced is not None
    if has_splits != (dDTS is not None):
        raise ValueError("DTS_reduced and dDTS must be given together")
    dts = dd = None
    if has_splits:
        dts, dd = DTS_reduced.contiguous(), dDTS.contiguous()
        for name, t in (("DTS_reduced", dts), ("dDTS", dd)):
            if tuple(t.shape) != (W, S) or t.dtype != dt:
                raise ValueError(f"{name} must be a [W, S] tensor of the Pi dtype")
    cs = []
    for c in consts:
        t = H.f(c, dt, dev)
        cs.append(t.reshape(1, -1) if t.ndim == 1 else t)
    shape = tuple(cs[2].shape)
    cs = [c if tuple(c.shape) == shape else c.expand(*shape).contiguous() for c in cs]
    mt, dmc, DL, dDL, Eb, dEb, Ev, dEv, SL1, dSL1, SL2, dSL2 = cs
    tree = H.tree_from_parent(node_parent, node_child1, node_child2)
    col = H.f(col_log_probs, dt, dev)
    item = H.i64(item_idx, dev)
    leaf = H.i64(leaf_state_idx, dev)
    lp, dlp = H.f(leaf_logp, dt, dev), H.f(dleaf_logp, dt, dev)
    io = H.KbWaveTanIO(
        dtype=H.dtype_code(dt), S=S, W=W, use_col_weights=int(bool(use_col_weights)),
        use_leaf_index=int(bool(has_leaf_term)), n_iters=max(1, int(n_iters)), ws=ws, pi_ws=int(pi_ws),
        const_stride=_const_stride(DL), Pi_in=H.ptr(Pi_in), dPi_in=H.ptr(dPi_in), dPi_out=H.ptr(dPi_out),
        dPibar_out=H.ptr(dPibar_out), dts=H.ptr(dts), d_dts=H.ptr(dd), max_coupling=H.ptr(mt), dMC=H.ptr(dmc),
        DL=H.ptr(DL), dDL=H.ptr(dDL), Ebar=H.ptr(Eb), dEbar=H.ptr(dEb), E=H.ptr(Ev), dE=H.ptr(dEv),
        SL1=H.ptr(SL1), dSL1=H.ptr(dSL1), SL2=H.ptr(SL2), dSL2=H.ptr(dSL2), col_log_probs=H.ptr(col),
        item_idx=H.ptr(item), leaf_state=H.ptr(leaf), leaf_logp=H.ptr(lp), dleaf_logp=H.ptr(dlp),
    )
    H.check(H.lib().kb_wave_step_tangent(tree.handle, io, H.stream(dev)))
    H.wrote(dPi_out, dPibar_out)


def compute_wave_step_tangent_selfloop(Pi_in, dPi_io, ws, W, S, n_iters, max_coupling_mat, dMC, DL, dDL, Ebar, dEbar,
                                       E, dE, SL1, dSL1, SL2, dSL2, col_log_probs, node_child1, node_child2,
                                       node_parent, max_ancestor_depth, DTS_reduced=None, dDTS=None, *,
                                       leaf_state_idx, leaf_logp, dleaf_logp, item_idx, dPibar_out=None,
                                       has_leaf_term=True, use_col_weights=True):
    """``n_iters`` in-place tangent sweeps of rows [ws, ws + W) of ``dPi_io`` in one launch
    (reference wave_tangent.py:346-389); ``dPibar_out[ws:ws+W]`` gets the last sweep's dPibar."""
    _launch(Pi_in, dPi_io, dPi_io, ws, W, S, n_iters, ws,
            (max_coupling_mat, dMC, DL, dDL, Ebar, dEbar, E, dE, SL1, dSL1, SL2, dSL2), col_log_probs, node_child1,
            node_child2, node_parent, DTS_reduced, dDTS, leaf_state_idx, leaf_logp, dleaf_logp, item_idx, dPibar_out,
            has_leaf_term, use_col_weights, "compute_wave_step_tangent_selfloop")


def compute_wave_step_tangent(Pi_in, dPi_in, dPi_out, ws, W, S, max_coupling_mat, dMC, DL, dDL, Ebar, dEbar, E, dE,
                              SL1, dSL1, SL2, dSL2, col_log_probs, node_child1, node_child2, node_parent,
                              max_ancestor_depth, DTS_reduced=None, dDTS=None, *, leaf_state_idx, leaf_logp,
                              dleaf_logp, item_idx, dPibar_out=None, has_leaf_term=True, input_ws=None,
                              use_col_weights=True):
    """One tangent sweep: rows [ws, ws + W) of ``dPi_out`` from primal / tangent rows
    ``input_ws + w`` (default ``ws``) of ``Pi_in`` / ``dPi_in`` (reference wave_tangent.py:392-431)."""
    _launch(Pi_in, dPi_in, dPi_out, ws, W, S, 1, int(ws) if input_ws is None else int(input_ws),
            (max_coupling_mat, dMC, DL, dDL, Ebar, dEbar, E, dE, SL1, dSL1, SL2, dSL2), col_log_probs, node_child1,
            node_child2, node_parent, DTS_reduced, dDTS, leaf_state_idx, leaf_logp, dleaf_logp, item_idx, dPibar_out,
            has_leaf_term, use_col_weights, "compute_wave_step_tangent")
