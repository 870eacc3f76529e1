"""Wave-sweep wrappers on the HIP kernels (drop-in for the reference kbench/core/kernels/wave_step.py).

* ``compute_leaf_initial_wave_step`` -- leaf initialisation of a wave
  (reference pristine wave_step.py:313-361);
* ``compute_wave_step`` -- one self-loop sweep of a wave, optionally with the
  split term, the final Pibar / row max and the per-row residual (reference
  pristine wave_step.py:363-410).

Same positional / keyword signatures and in-place semantics: rows
[ws, ws + W) of ``Pi_out`` (and of ``Pibar`` / ``pibar_row_max`` with
``store_final_pibar``) are written, ``Pi_out is Pibar`` and ``Pi_in`` being the
[W, S] split buffer (``input_ws=0``) are allowed.  One 1024-thread workgroup
per row; the Pibar ancestor sums are one Euler-tour prefix scan in LDS instead
of the reference's bounded ancestor chase (same sum).
"""

from __future__ import annotations

import torch

from . import _hip as H

__all__ = ["compute_leaf_initial_wave_step", "compute_wave_step"]


def _const_stride(c) -> int:
    """0 for one shared constant row, else the row stride (reference wave_step.py:10-13)."""
    return 0 if int(c.shape[0]) == 1 else int(c.stride(0))


def _consts(dt, dev, *cs):
    out = []
    for c in cs:
        t = H.f(c, dt, dev)
        out.append(t.reshape(1, -1) if t.ndim == 1 else t)
    return out


def compute_leaf_initial_wave_step(Pi_out, ws, W, S, max_coupling_mat, DL_const, Ebar, E, SL1_const, SL2_const,
                                   col_log_probs, node_child1, node_child2, node_subtree_start, node_subtree_end,
                                   leaf_state_idx, leaf_logp, item_idx, use_col_weights=True):
    """Leaf initialisation of rows [ws, ws + W) into Pi_out (reference wave_step.py:313-361)."""
    W, S, ws = int(W), int(S), int(ws)
    if W <= 0:
        return
    H.require_device(Pi_out, "compute_leaf_initial_wave_step")
    dt, dev = Pi_out.dtype, Pi_out.device
    if not Pi_out.is_contiguous() or int(Pi_out.shape[1]) != S:
        raise ValueError("Pi_out must be a contiguous [C, S] tensor")
    mt, DL, Eb, Ev, SL1, SL2 = _consts(dt, dev, max_coupling_mat, DL_const, Ebar, E, SL1_const, SL2_const)
    keep = dict(mt=mt, DL=DL, Eb=Eb, Ev=Ev, SL1=SL1, SL2=SL2, col=H.f(col_log_probs, dt, dev),
                c1=H.i64(node_child1, dev), c2=H.i64(node_child2, dev), ss=H.i64(node_subtree_start, dev),
                se=H.i64(node_subtree_end, dev), item=H.i64(item_idx, dev), leaf=H.i64(leaf_state_idx, dev),
                lp=H.f(leaf_logp, dt, dev))
    io = H.KbLeafInitIO(
        dtype=H.dtype_code(dt), S=S, W=W, use_col_weights=int(bool(use_col_weights)), ws=ws,
        const_stride=_const_stride(DL), node_child1=H.ptr(keep["c1"]), node_child2=H.ptr(keep["c2"]),
        Pi_out=H.ptr(Pi_out), max_coupling=H.ptr(mt), DL=H.ptr(DL), Ebar=H.ptr(Eb), E=H.ptr(Ev), SL1=H.ptr(SL1),
        SL2=H.ptr(SL2), col_log_probs=H.ptr(keep["col"]), subtree_start=H.ptr(keep["ss"]),
        subtree_end=H.ptr(keep["se"]), item_idx=H.ptr(keep["item"]), leaf_state=H.ptr(keep["leaf"]),
        leaf_logp=H.ptr(keep["lp"]),
    )
    H.check(H.lib().kb_leaf_init(io, H.stream(dev)))


def compute_wave_step(Pi_in, Pi_out, Pibar, ws, W, S, max_coupling_mat, DL_const, Ebar, E, SL1_const, SL2_const,
                      col_log_probs, node_child1, node_child2, node_parent, max_ancestor_depth, DTS_reduced=None, *,
                      leaf_state_idx, leaf_logp, item_idx, pibar_row_max, store_final_pibar=False,
                      has_leaf_term=True, input_ws=None, use_col_weights=True, pi_residual_out=None):
    """One self-loop sweep of rows [ws, ws + W) (reference wave_step.py:363-410).

    Input row w is ``Pi_in[input_ws + w]`` (``input_ws`` defaults to ``ws``);
    the new row goes to ``Pi_out[ws + w]``.  ``DTS_reduced`` [W, S] adds the
    split term; ``has_leaf_term`` the leaf observation term.
    ``store_final_pibar`` also writes ``Pibar[ws + w]`` and
    ``pibar_row_max[ws + w]`` from the new row; ``pi_residual_out`` (float32
    [C]) receives max |Pi_new - Pi_in| over finite entries.
    """
    W, S, ws = int(W), int(S), int(ws)
    if W <= 0:
        return
    H.require_device(Pi_in, "compute_wave_step")
    dt, dev = Pi_in.dtype, Pi_in.device
    for name, t in (("Pi_in", Pi_in), ("Pi_out", Pi_out), ("Pibar", Pibar)):
        if not t.is_contiguous() or t.ndim != 2 or int(t.shape[1]) != S:
            raise ValueError(f"{name} must be a contiguous [*, S] tensor")
        if t.dtype != dt:
            raise RuntimeError(f"{name} has dtype {t.dtype}, expected {dt}")
    if pibar_row_max.dtype != dt or not pibar_row_max.is_contiguous():
        raise ValueError("pibar_row_max must be a contiguous tensor of the Pi dtype")
    if pi_residual_out is not None and (pi_residual_out.dtype != torch.float32
                                        or not pi_residual_out.is_contiguous()):
        raise ValueError("pi_residual_out must be a contiguous float32 tensor")
    dts = None
    if DTS_reduced is not None:
        dts = DTS_reduced
        if not dts.is_contiguous() or tuple(dts.shape) != (W, S) or dts.dtype != dt:
            raise ValueError("DTS_reduced must be a contiguous [W, S] tensor of the Pi dtype")
    tree = H.tree_from_parent(node_parent, node_child1, node_child2)
    mt, DL, Eb, Ev, SL1, SL2 = _consts(dt, dev, max_coupling_mat, DL_const, Ebar, E, SL1_const, SL2_const)
    col = H.f(col_log_probs, dt, dev)
    item = H.i64(item_idx, dev)
    leaf = H.i64(leaf_state_idx, dev)
    lp = H.f(leaf_logp, dt, dev)
    io = H.KbWaveStepIO(
        dtype=H.dtype_code(dt), S=S, W=W, use_col_weights=int(bool(use_col_weights)),
        use_leaf_index=int(bool(has_leaf_term)), store_final_pibar=int(bool(store_final_pibar)), ws=ws,
        pi_ws=ws if input_ws is None else int(input_ws), const_stride=_const_stride(DL),
        Pi_in=H.ptr(Pi_in), Pi_out=H.ptr(Pi_out), Pibar=H.ptr(Pibar), pibar_row_max=H.ptr(pibar_row_max),
        pi_residual=H.ptr(pi_residual_out), dts=H.ptr(dts), max_coupling=H.ptr(mt), DL=H.ptr(DL), Ebar=H.ptr(Eb),
        E=H.ptr(Ev), SL1=H.ptr(SL1), SL2=H.ptr(SL2), col_log_probs=H.ptr(col), item_idx=H.ptr(item),
        leaf_state=H.ptr(leaf), leaf_logp=H.ptr(lp),
    )
    H.check(H.lib().kb_wave_step(tree.handle, io, H.stream(dev)))
