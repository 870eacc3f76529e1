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

Launch collapse (``KBENCH_FUSE_SWEEPS=1``).  A caller that sweeps a wave
``pi_iters - 1`` times (reference kbench/core/inference/forward.py:81-115)
issues one call per sweep, each reading the previous call's ``Pi_out``.
With the variable set, a call without ``store_final_pibar`` that continues
such a chain (same rows, constants and split term; its ``Pi_in`` is the
previous call's ``Pi_out``) is held back, and the chain runs as one launch of
``n`` sweeps with the row on chip when its final call arrives: the same
final Pi, Pibar, row maxima and residual up to float32 rounding (a float
chain runs in linear space at preorder positions, with its path sums added in
another order; float64 chains are bitwise those of single sweeps).  Held-back calls leave their
own ``Pi_out`` rows unwritten: a caller must not read a chain's intermediate
buffers before its final call (the reference glue never does).  Any other
wrapper call, or a call that breaks the chain, first runs what is held back.
"""

from __future__ import annotations

import os

import torch

from . import _hip as H

FUSE_SWEEPS = os.environ.get("KBENCH_FUSE_SWEEPS", "0").strip() not in ("", "0")

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
    H.wrote(Pi_out)


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
    pi_ws = ws if input_ws is None else int(input_ws)
    # the chain identity: everything a held-back sweep shares with the next one
    key = (ws, W, S, dt, dev, bool(has_leaf_term), bool(use_col_weights), dts, max_coupling_mat, DL_const, Ebar,
           E, SL1_const, SL2_const, col_log_probs, node_parent, node_child1, node_child2, item_idx, leaf_state_idx,
           leaf_logp)
    chain = _chain
    if chain is not None and not chain.continued_by(key, Pi_in, pi_ws):
        H.flush()  # runs and clears the held-back chain
        chain = None
    if FUSE_SWEEPS and not store_final_pibar and pi_residual_out is None:
        if chain is None:
            chain = _Chain(key, Pi_in, pi_ws)
        chain.extend(Pi_out, Pibar, pibar_row_max)
        _hold(chain)
        return
    first_in, first_ws, n_held = (chain.first_in, chain.first_ws, chain.n) if chain is not None else (Pi_in, pi_ws, 0)
    _drop_held()
    _launch_sweeps(first_in, first_ws, n_held + 1, Pi_out, Pibar, pibar_row_max, pi_residual_out,
                   bool(store_final_pibar), key, dts)


class _Chain:
    """Sweeps of one wave held back under KBENCH_FUSE_SWEEPS, waiting for the chain's final call."""

    __slots__ = ("key", "first_in", "first_ws", "n", "last_out", "last_pibar", "last_rmax")

    def __init__(self, key, Pi_in, pi_ws):
        self.key, self.first_in, self.first_ws, self.n = key, Pi_in, pi_ws, 0
        self.last_out = self.last_pibar = self.last_rmax = None

    def extend(self, Pi_out, Pibar, rmax):
        self.n += 1
        self.last_out, self.last_pibar, self.last_rmax = Pi_out, Pibar, rmax

    def continued_by(self, key, Pi_in, pi_ws) -> bool:
        """The next sweep reads this chain's last output rows with the same rows and constants."""
        if Pi_in is not self.last_out or pi_ws != key[0] or len(key) != len(self.key):
            return False
        return all(a is b or (type(a) is type(b) and not torch.is_tensor(a) and a == b)
                   for a, b in zip(key, self.key))

    def run(self):
        """Launch the held-back sweeps alone (a chain broken before its final call)."""
        _launch_sweeps(self.first_in, self.first_ws, self.n, self.last_out, self.last_pibar, self.last_rmax,
                       None, False, self.key, self.key[7])


_chain = None


def _hold(chain):
    global _chain
    _chain = chain
    H.defer(_run_held)


def _run_held():
    global _chain
    chain, _chain = _chain, None
    if chain is not None:
        chain.run()


def _drop_held():
    global _chain
    if _chain is not None:
        _chain = None
        H.defer(None)


def _launch_sweeps(Pi_in, pi_ws, n_sweeps, Pi_out, Pibar, pibar_row_max, pi_residual_out, store_final, key, dts):
    """One kb_wave_step launch of ``n_sweeps`` sweeps from ``Pi_in`` rows ``pi_ws..``."""
    (ws, W, S, dt, dev, has_leaf, use_col, _, mt_c, DL_c, Ebar_c, E_c, SL1_c, SL2_c, col_c, parent, c1, c2, item_c,
     leaf_c, lp_c) = key
    tree = H.tree_from_parent(parent, c1, c2)
    mt, DL, Eb, Ev, SL1, SL2 = _consts(dt, dev, mt_c, DL_c, Ebar_c, E_c, SL1_c, SL2_c)
    col = H.f(col_c, dt, dev)
    item = H.i64(item_c, dev)
    leaf = H.i64(leaf_c, dev)
    lp = H.f(lp_c, dt, dev)
    io = H.KbWaveStepIO(
        dtype=H.dtype_code(dt), S=S, W=W, use_col_weights=int(use_col), use_leaf_index=int(has_leaf),
        store_final_pibar=int(store_final), n_sweeps=int(n_sweeps), ws=ws, pi_ws=int(pi_ws),
        const_stride=_const_stride(DL), Pi_in=H.ptr(Pi_in), Pi_out=H.ptr(Pi_out), Pibar=H.ptr(Pibar),
        pibar_row_max=H.ptr(pibar_row_max), pi_residual=H.ptr(pi_residual_out), dts=H.ptr(dts),
        max_coupling=H.ptr(mt), DL=H.ptr(DL), Ebar=H.ptr(Eb), E=H.ptr(Ev), SL1=H.ptr(SL1), SL2=H.ptr(SL2),
        col_log_probs=H.ptr(col), item_idx=H.ptr(item), leaf_state=H.ptr(leaf), leaf_logp=H.ptr(lp),
    )
    H.check(H.N.lib().kb_wave_step(tree.handle, io, H.stream(dev)))
    H.wrote(Pi_out, Pibar if store_final else None, pibar_row_max if store_final else None, pi_residual_out)
