"""Oracle-backed stand-ins for the per-call wrappers: the independent side of the replay gate.

Each stand-in has the signature of the ``kbench.core.kernels`` wrapper it
replaces (arguments are bound through that wrapper's own signature), reads
the call's device tensors, computes the reference kernel's outputs with the
float64 CPU oracle, and writes them back the way the wrapper does: rows
[ws, ws + W) of the caller's buffers in place, accumulators incremented,
fresh tensors returned.  ``capture.replay(record, pool, fn=stand_in)`` then
compares the oracle's outputs on a recorded call's own inputs with that call's
recorded HIP outputs, as the reference's gate compares a candidate with
captured pristine outputs (reference capture/capture.py:164-210,
bench/kernels.py:54-94).

Test infrastructure only.  The stand-ins cover the argument patterns of the
per-call solve (``kbench.percall``): one parameter row (item_rows == 1),
uniform or weighted columns, Neumann or GMRES self-loop solves; anything else
raises ``NotImplementedError``.
"""

from __future__ import annotations

import inspect

import numpy as np
import torch

import kbench_oracle as O


def _h(t):
    """Host float64 / int64 copy of a tensor (None stays None)."""
    if t is None:
        return None
    if not torch.is_tensor(t):
        return np.asarray(t)
    t = t.detach().cpu()
    return t.double().numpy() if t.is_floating_point() else t.long().numpy()


def _put(dst, rows, val):
    """dst[rows] = val (host float64 -> dst's dtype and device)."""
    dst[rows] = torch.as_tensor(np.asarray(val), dtype=dst.dtype, device=dst.device)


def _add(dst, val):
    dst.add_(torch.as_tensor(np.asarray(val).reshape(dst.shape), dtype=dst.dtype, device=dst.device))


def _state_rows(t, S):
    """A [G, S] host copy of an item-state constant."""
    a = _h(t)
    return np.broadcast_to(a.reshape(-1, S) if a.size % S == 0 else a.reshape(-1, 1), (max(1, a.size // S), S)).copy()


def _param(t, S):
    """The oracle's [G, S] or [G, 1] parameter row of a per-state or global parameter."""
    a = _h(t)
    return a.reshape(1, -1) if a.size in (1, S) else a.reshape(-1, a.shape[-1])


def _consts(a, S, leaf_logp, col, use_col):
    return O.WaveConsts(mt=_state_rows(a["max_coupling_mat"] if "max_coupling_mat" in a else a["mt_squeezed"], S),
                        DL=_state_rows(a["DL_const"], S), Ebar=_state_rows(a["Ebar"], S), E=_state_rows(a["E"], S),
                        SL1=_state_rows(a["SL1_const"], S), SL2=_state_rows(a["SL2_const"], S),
                        leaf_logp=None if leaf_logp is None else _state_rows(leaf_logp, S), col=_h(col).reshape(-1),
                        use_col_weights=bool(use_col))


class OracleWrappers:
    """The stand-ins, bound to one species tree (``O.Tree``)."""

    def __init__(self, tree: O.Tree):
        self.tree = tree

    @staticmethod
    def _bind(name, args, kwargs):
        from kbench.capture import WRAPPERS
        import importlib

        real = getattr(importlib.import_module(WRAPPERS[name]), name)
        b = inspect.signature(real).bind(*args, **kwargs)
        b.apply_defaults()
        return b.arguments

    def fn(self, name):
        return getattr(self, name)

    # ------------------------------------------------------------------ forward
    def compute_leaf_initial_wave_step(self, *args, **kwargs):
        a = self._bind("compute_leaf_initial_wave_step", args, kwargs)
        ws, W, S = int(a["ws"]), int(a["W"]), int(a["S"])
        rows = np.arange(ws, ws + W)
        oc = _consts(a, S, a["leaf_logp"], a["col_log_probs"], a["use_col_weights"])
        items = _h(a["item_idx"])[rows]
        _put(a["Pi_out"], slice(ws, ws + W), O.leaf_initial(_h(a["leaf_state_idx"])[rows], items, oc, self.tree))

    def compute_wave_step(self, *args, **kwargs):
        a = self._bind("compute_wave_step", args, kwargs)
        if a["pi_residual_out"] is not None:
            raise NotImplementedError("pi_residual_out")
        ws, W, S = int(a["ws"]), int(a["W"]), int(a["S"])
        rows = np.arange(ws, ws + W)
        src_ws = ws if a["input_ws"] is None else int(a["input_ws"])
        src = _h(a["Pi_in"])[src_ws:src_ws + W]
        oc = _consts(a, S, a["leaf_logp"], a["col_log_probs"], a["use_col_weights"])
        items = _h(a["item_idx"])[rows]
        leaf = _h(a["leaf_state_idx"])[rows] if a["has_leaf_term"] else None
        dts = _h(a["DTS_reduced"])
        new = O.wave_sweep(src, items, oc, self.tree, leaf_state=leaf, dts_r=dts)
        _put(a["Pi_out"], slice(ws, ws + W), new)
        if a["store_final_pibar"]:
            pb, rm = O._pibar_from_pi(new, oc.col, oc.mt[items], self.tree, oc.use_col_weights)
            _put(a["Pibar"], slice(ws, ws + W), pb)
            _put(a["pibar_row_max"], slice(ws, ws + W), rm)

    def compute_dts_forward(self, *args, **kwargs):
        a = self._bind("compute_dts_forward", args, kwargs)
        Pi = a["Pi"]
        S, W = int(Pi.shape[1]), int(a["W"])
        meta = {"sl": _h(a["lefts"]), "sr": _h(a["rights"]), "reduce_idx": _h(a["reduce_idx"])}
        if a["log_split_probs"] is not None:
            meta["log_split_probs"] = _h(a["log_split_probs"])
        act = None if a["active_parent_rows"] is None else _h(a["active_parent_rows"]).astype(bool)
        out = O.dts_forward(_h(Pi), _h(a["Pibar"]), meta, W, _param(a["log_pD_vec"], S), _param(a["log_pS_vec"], S),
                            _h(a["item_idx"]), int(a["item_offset"]), self.tree, active=act)
        return torch.as_tensor(out, dtype=Pi.dtype, device=Pi.device)

    def e_fixed_point_triton(self, *args, **kwargs):
        a = self._bind("e_fixed_point_triton", args, kwargs)
        E0 = a["E0"]
        G, S = (int(E0.shape[0]), int(E0.shape[1])) if E0.ndim == 2 else (1, int(E0.numel()))
        st = lambda t: O.as_item_state(_h(t), S, G)
        out = O.e_fixed_point(_h(E0).reshape(G, S), st(a["log_pS"]), st(a["log_pD"]), st(a["log_pL"]),
                              st(a["max_coupling"]), _h(a["col_log_probs"]).reshape(-1), self.tree,
                              bool(a["use_col_weights"]), int(a["max_iter"]), float(a["tol"]))
        return tuple(torch.as_tensor(x, dtype=E0.dtype, device=E0.device).reshape(E0.shape) for x in out[:4])

    # ------------------------------------------------------------------ backward
    def active_mask_from_rhs_absmax_fused(self, *args, **kwargs):
        a = self._bind("active_mask_from_rhs_absmax_fused", args, kwargs)
        rhs = a["rhs"]
        m = O.active_mask(_h(rhs), float(a["threshold"]), bool(a["use_pruning"]))
        return torch.as_tensor(m, dtype=torch.bool, device=rhs.device)

    def wave_backward_uniform_fused(self, *args, **kwargs):
        a = self._bind("wave_backward_uniform_fused", args, kwargs)
        if a["self_loop_grad_targets"] is not None or a["initial_v"] is not None or a["return_last_increment"]:
            raise NotImplementedError("self_loop_grad_targets / initial_v / return_last_increment")
        ws, W, S = int(a["ws"]), int(a["W"]), int(a["S"])
        rows = np.arange(ws, ws + W)
        Pi = a["Pi_star"]
        use_leaf = bool(a["has_leaf_term"]) and a["leaf_state_idx"] is not None and a["leaf_logp"] is not None
        oc = _consts(a, S, a["leaf_logp"], a["col_log_probs"], a["use_col_weights"])
        items = _h(a["item_idx"])[rows]
        act = (np.ones(W, dtype=bool) if a["active_mask"] is None else _h(a["active_mask"]).astype(bool))
        out = O.wave_backward_uniform(_h(Pi)[rows], _h(a["Pibar_star"])[rows], _h(a["pibar_row_max"])[rows],
                                      _h(a["rhs"]), items, oc, self.tree, int(a["neumann_terms"]), active=act,
                                      leaf_state=_h(a["leaf_state_idx"])[rows] if use_leaf else None,
                                      dts_r=_h(a["dts_r"]), solver=str(a["self_loop_solver"]).strip().lower())
        if a["grad_col_log_probs"] is not None:
            _add(a["grad_col_log_probs"], out[7])
        return tuple(torch.as_tensor(x, dtype=Pi.dtype, device=Pi.device) for x in out[:7])

    def dts_cross_backward_accum_fused(self, *args, **kwargs):
        a = self._bind("dts_cross_backward_accum_fused", args, kwargs)
        if not (a["output_pibar_ud"] and a["output_pibar_side_active"] and a["accum_param_reductions"]
                and a["accum_mt_reduction"]):
            raise NotImplementedError("the per-call solve's option set only")
        Pi = a["Pi_star"]
        S, ws = int(a["S"]), int(a["ws"])
        meta = {"sl": _h(a["sl"]), "sr": _h(a["sr"]), "reduce_idx": _h(a["reduce_idx"]),
                "log_split_probs": _h(a["wlsp"]).reshape(-1)}
        v = _h(a["v_k"])
        W = int(v.shape[0])
        act_w = np.ones(W, dtype=bool) if a["active_mask"] is None else _h(a["active_mask"]).astype(bool)
        thr = float(a["pibar_side_threshold"])
        mt = _state_rows(a["mt_squeezed"], S)
        col = np.zeros(S)  # the direct rows, u_d and the sums below do not read the column weights
        r = O.dts_cross_backward(_h(Pi), _h(a["Pibar_star"]), _h(a["pibar_row_max"]), v, ws, meta,
                                 _param(a["log_pD"], S), _param(a["log_pS"], S), mt, _h(a["item_idx"]), self.tree,
                                 act_w, col, False, side_thr=thr)
        acc = a["accumulated_rhs"]
        dirs = np.zeros((acc.shape[0], S))
        np.add.at(dirs, meta["sl"], r["direct_l"])
        np.add.at(dirs, meta["sr"], r["direct_r"])
        _add(acc, dirs)
        _add(a["grad_log_pD"], r["g_pD"].sum(axis=0).reshape(a["grad_log_pD"].shape) if a["grad_log_pD"].numel() == S
             else r["g_pD"].sum())
        _add(a["grad_log_pS"], r["g_pS"].sum(axis=0).reshape(a["grad_log_pS"].shape) if a["grad_log_pS"].numel() == S
             else r["g_pS"].sum())
        gmt = r["g_mt_l"].sum(axis=0) + r["g_mt_r"].sum(axis=0)
        _add(a["grad_mt"], gmt if a["grad_mt"].numel() == S else gmt.sum())
        ud = np.concatenate([r["ud_l"], r["ud_r"]])
        A = np.concatenate([r["A_l"], r["A_r"]])
        on = np.concatenate([r["active_split"], r["active_split"]])
        if thr > 0.0:
            side = on & (np.abs(ud).sum(axis=1) > thr)
        else:
            side = on & (np.abs(ud).max(axis=1, initial=0.0) != 0.0)
        t = lambda x: torch.as_tensor(x, dtype=Pi.dtype, device=Pi.device)
        return t(ud), t(A), torch.as_tensor(side, dtype=torch.bool, device=Pi.device), None, None

    def uniform_cross_pibar_vjp_tree_from_ud_fused(self, *args, **kwargs):
        a = self._bind("uniform_cross_pibar_vjp_tree_from_ud_fused", args, kwargs)
        if a["side_active"] is None:
            raise NotImplementedError("the per-call solve passes side_active")
        Pi = a["Pi_star"]
        S = int(a["S"])
        sl, sr = _h(a["sl"]), _h(a["sr"])
        n = sl.shape[0]
        child = np.concatenate([sl, sr])
        side = _h(a["side_active"]).astype(bool)
        if a["active_mask"] is not None:
            act = _h(a["active_mask"]).astype(bool)[_h(a["reduce_idx"])]
            side = side & np.concatenate([act, act])
        ud = _h(a["pibar_ud"])
        A = _h(a["pibar_A"]).reshape(-1)
        sub = self.tree.subtree_sum(ud)
        Pi_h, rmax = _h(Pi), _h(a["pibar_row_max"])
        wPi = Pi_h[child] + _h(a["col_log_probs"]).reshape(1, -1) if a["use_col_weights"] else Pi_h[child]
        pp = np.exp2(wPi - O._safe(rmax[child])[:, None])
        contrib = np.where(side[:, None], pp * (A[:, None] - sub), 0.0)
        ud_new = np.where(side[:, None], sub, ud)
        _put(a["pibar_ud"], slice(0, 2 * n), ud_new)
        acc = a["accumulated_rhs"]
        rows = np.zeros((acc.shape[0], S))
        np.add.at(rows, child, contrib)
        _add(acc, rows)
        if a["grad_col_log_probs"] is not None:
            _add(a["grad_col_log_probs"], contrib.sum(axis=0))
        return a["side_active"]
