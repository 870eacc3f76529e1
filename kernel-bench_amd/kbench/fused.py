"""Whole-pass native driver: the MI355X fast path for ``run_forward`` / ``run_backward``.

``FusedSolver`` builds the device-resident layout tables once per static
problem (``kb_plan_create``) and then runs a whole forward or backward pass
with a handful of launches on the current stream:

* forward: one single-workgroup kernel for the parameters and the E-step fixed
  point, one fused kernel per wave (split reduction + all ``pi_iters-1`` sweeps
  + final Pibar), and a two-kernel deterministic loss reduction;
* backward: one fused kernel per wave in reverse order (child-owned gather of
  the adjoint, active mask, split recomputation, self-loop Neumann series,
  parameter buckets, split-side staging) and a final O(S) epilogue for the
  E adjoint and the theta / column VJP.

It computes what the reference's frozen glue computes
(reference kbench/runtime.py:63-115) and returns the same tensors;
``kbench.runtime`` exposes it under the reference's entry-point names.
"""

from __future__ import annotations

import ctypes as ct
import os
import weakref
from types import SimpleNamespace

import numpy as np
import torch

from . import _native as N

# Default early-stop tolerance of the backward's Neumann series: 2^-24,
# float32's unit roundoff, relative to the row's largest right-hand-side entry.
# Every adjoint entry has one sign and the terms decay geometrically (by about
# 5-10x per term at config 3), so the dropped remainder is of that order
# relative to the row's adjoints: gradients move by about 1e-7 relative, the
# size of float32 rounding of the sums, while a row needs about half of its
# 16 terms.
DEFAULT_NEUMANN_RTOL = 2.0 ** -24

FORWARD_SAVED_NAMES = (
    "E", "E_s1", "E_s2", "Ebar", "root_rows", "pi_wave", "pibar_wave",
    "pibar_row_max", "log_pS", "log_pD", "log_pL", "max_coupling", "col_log_probs",
)

_SOLVER_DEFAULTS = {
    "e_init": -1.0, "e_max_iter": 2000, "e_tol": 1e-8, "pi_iters": 6, "neumann_terms": 3,
    "self_loop_solver": "neumann", "bicgstab_max_iter": 500, "bicgstab_tol": 1e-7,
    "bicgstab_breakdown_tol": 1e-30, "adjoint_pruning_threshold": 1e-6,
    "use_adjoint_pruning": True, "pibar_side_threshold": 0.0,
}


class _TensorKey:
    """Identity of a live tensor object and its in-place version counter.

    Holds a weak reference, so a key never matches a different tensor that was
    later allocated at the freed address (the object identity is checked, not
    the address), and never keeps the tensor alive.
    """

    __slots__ = ("ref", "version")

    def __init__(self, t):
        self.ref = weakref.ref(t)
        self.version = int(t._version)

    def matches(self, t) -> bool:
        return self.ref() is t and int(t._version) == self.version


def _np(x, dtype=None):
    if torch.is_tensor(x):
        x = x.detach().cpu().numpy()
    a = np.asarray(x)
    return a.astype(dtype) if dtype is not None else a


def _get(static, key):
    return static[key] if isinstance(static, dict) else getattr(static, key)


def solver_options_dict(so) -> dict:
    d = dict(_SOLVER_DEFAULTS)
    if so is None:
        return d
    if isinstance(so, dict):
        d.update(so)
    else:
        for k in d:
            if hasattr(so, k):
                d[k] = getattr(so, k)
    return d


def layout_arrays(static) -> dict:
    """Host (numpy) arrays of the ``kb_layout`` struct from a ``static`` namespace or dict.

    Splits are flattened over the waves with their global parent row
    (wave start + reduce_idx); a wave without ``log_split_probs`` has 0.
    """
    wl = _get(static, "wave_layout")
    sh = _get(static, "state_helpers")
    ws, wsz, whs = [], [], []
    sp, sl, sr, lsp = [], [], [], []
    for m in wl["wave_metas"]:
        start, W = int(m["start"]), int(m["W"])
        ws.append(start)
        wsz.append(W)
        has = "sl" in m
        whs.append(1 if has else 0)
        if has:
            a = _np(m["sl"], np.int64)
            lp = m.get("log_split_probs")
            sp.append(_np(m["reduce_idx"], np.int64) + start)
            sl.append(a)
            sr.append(_np(m["sr"], np.int64))
            lsp.append(np.zeros(a.shape[0]) if lp is None else _np(lp, np.float64).reshape(-1))
    cat = lambda xs, dt: (np.concatenate(xs).astype(dt) if xs else np.zeros(0, dtype=dt))
    arrays = {
        "node_parent": _np(sh["node_parent"], np.int64),
        "node_child1": _np(sh["node_child1"], np.int64),
        "node_child2": _np(sh["node_child2"], np.int64),
        "node_subtree_start": _np(sh["node_subtree_start"], np.int64),
        "node_subtree_end": _np(sh["node_subtree_end"], np.int64),
        "unnorm_row_max": _np(sh["unnorm_row_max"], np.float32),
        "leaf_state_index": _np(wl["leaf_state_index"], np.int64),
        "rate_item_idx": _np(_get(static, "rate_item_idx"), np.int64),
        "root_row_ids": _np(wl["root_row_ids"], np.int64),
        "wave_start": np.asarray(ws, np.int64),
        "wave_size": np.asarray(wsz, np.int64),
        "wave_has_splits": np.asarray(whs, np.int32),
        "split_parent": cat(sp, np.int64),
        "split_left": cat(sl, np.int64),
        "split_right": cat(sr, np.int64),
        "split_log_prob": cat(lsp, np.float64),
    }
    arrays = {k: np.ascontiguousarray(v) for k, v in arrays.items()}
    arrays["S"] = int(_get(static, "state_helpers")["S"])
    return arrays


def kb_layout(arrays: dict) -> "N.KbLayout":
    """The ``kb_layout`` struct over ``arrays`` (the arrays must outlive the struct)."""
    L = N.KbLayout()
    L.S, L.C = int(arrays["S"]), int(arrays["leaf_state_index"].shape[0])
    L.n_fam, L.n_waves = int(arrays["root_row_ids"].shape[0]), int(arrays["wave_start"].shape[0])
    for k, v in arrays.items():
        if k == "S":
            continue
        if v.dtype == np.int64:
            setattr(L, k, v.ctypes.data_as(N.P_i64))
        elif v.dtype == np.int32:
            setattr(L, k, v.ctypes.data_as(N.P_i32))
        elif v.dtype == np.float32:
            setattr(L, k, v.ctypes.data_as(N.P_f32))
        else:
            setattr(L, k, v.ctypes.data_as(N.P_f64))
    L.n_splits = int(arrays["split_left"].shape[0])
    return L


class FusedSolver:
    """Native whole-pass solver bound to one static layout and one device."""

    def __init__(self, static, solver_options=None, device=None, *, neumann_rtol=None):
        self.statewise = bool(_get(static, "statewise"))
        # the Neumann series' early stop (``kb_backward_io.neumann_rtol``): a row's series
        # ends at its first term whose entries are all at most this fraction of the row's
        # largest adjoint entry; 0 sums every ``neumann_terms`` term, as the reference does
        if neumann_rtol is None:
            neumann_rtol = float(os.environ.get("KB_NEUMANN_RTOL", DEFAULT_NEUMANN_RTOL))
        if not 0.0 <= float(neumann_rtol) < 1.0:
            raise ValueError("neumann_rtol must be in [0, 1)")
        self.neumann_rtol = float(neumann_rtol)
        self.itemwise = bool(_get(static, "itemwise"))
        if self.itemwise:
            raise NotImplementedError("the fused driver covers item_rows == 1 (itemwise=False)")
        so = solver_options if solver_options is not None else (
            static.get("solver_options") if isinstance(static, dict) else getattr(static, "solver_options", None))
        self.so = solver_options_dict(so)
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        arrays = layout_arrays(static)
        if np.any(arrays["rate_item_idx"] != 0):
            raise NotImplementedError("the fused driver needs rate_item_idx == 0 (itemwise=False)")
        self._arrays = arrays
        L = kb_layout(arrays)
        S, C, roots, ws = L.S, L.C, arrays["root_row_ids"], arrays["wave_start"]
        lib = N.lib()
        handle = ct.c_void_p()
        with torch.cuda.device(self.device):
            N.check(lib.kb_plan_create(ct.byref(L), ct.byref(handle)))
        self._plan = handle
        self.S, self.C, self.n_fam = S, C, int(roots.shape[0])
        self.root_row_ids = torch.as_tensor(roots, device=self.device)
        self.n_waves = len(ws)
        self.n_splits = L.n_splits
        info = (ct.c_int32 * 13)()
        N.check(lib.kb_plan_info(handle, info, 13))
        self.n_levels = int(info[6])
        # row classes: the forward computes one row per class of identical rows;
        # the backward solves every split row and one row per class of level-0 rows
        self.n_forward_rows = int(info[7])
        self.n_backward_rows = C - int(info[9]) + int(info[8])
        # solve(): the dependency level up to which whole families' backward rows run beside
        # the forward's later levels (-1: none), how many rows that is, and the lowest level
        # of those early launches (the levels below run whole afterwards)
        self.overlap_cut, self.overlap_rows, self.overlap_low = int(info[10]), int(info[11]), int(info[12])
        self.last_n_e_iter = None
        self.last_n_bicgstab = None
        self._use_col_cache = None  # (_TensorKey of the caller's col_weights, answer)
        self._last_forward = None   # (forward token, _TensorKey of pi, _TensorKey of pibar)

    def close(self):
        if getattr(self, "_plan", None):
            N.release("kb_plan_destroy", self._plan)  # held back while a graph capture is underway
            self._plan = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------------
    def _use_col(self, col_weights) -> bool:
        """True unless every column weight is equal (then the uniform fast path applies).

        ``col_weights`` is the caller's tensor (before any dtype / device
        conversion).  The answer is cached for that live tensor object and its
        version, so repeated solves with the same weights do not synchronise
        the host with the device; any other tensor is evaluated afresh.
        """
        hit = self._use_col_cache
        if hit is not None and hit[0].matches(col_weights):
            return hit[1]
        flat = col_weights.detach().reshape(-1)
        val = not bool(torch.all(flat == flat[0]).item())
        self._use_col_cache = (_TensorKey(col_weights), val)
        return val

    def run_forward(self, theta, col_weights, *, use_col_weights=None):
        """theta -> (loss, saved), the reference ``run_forward`` contract."""
        io, loss, saved, keep = self._forward_args(theta, col_weights, use_col_weights)
        with torch.cuda.device(self.device):
            N.check(N.lib().kb_forward(self._plan, ct.byref(io), N.stream_handle(self.device)))
        self._forward_done(saved)
        return loss, saved

    def _forward_done(self, saved):
        # the backward may reuse this forward's stored split terms while pi / pibar are
        # these same, unmodified tensor objects
        self._last_forward = (int(N.lib().kb_forward_token(self._plan)), _TensorKey(saved["pi_wave"]),
                              _TensorKey(saved["pibar_wave"]))

    def _forward_args(self, theta, col_weights, use_col_weights):
        """(kb_forward_io, loss, saved, kept tensors) of one forward: its outputs allocated, not run."""
        so = self.so
        dev = self.device
        S, C = self.S, self.C
        theta = theta.detach().to(device=dev, dtype=torch.float32).contiguous()
        use_col = self._use_col(col_weights) if use_col_weights is None else bool(use_col_weights)
        col_weights = col_weights.detach().to(device=dev, dtype=torch.float32).contiguous()
        if self.statewise and tuple(theta.shape) != (S, 3):
            raise ValueError(f"statewise theta must have shape ({S}, 3), got {tuple(theta.shape)}")
        if not self.statewise and tuple(theta.shape) != (3,):
            raise ValueError(f"theta must have shape (3,), got {tuple(theta.shape)}")
        f32 = dict(device=dev, dtype=torch.float32)
        E, E_s1, E_s2, Ebar = (torch.empty((1, S), **f32) for _ in range(4))
        npar = S if self.statewise else 1
        pS, pD, pL = (torch.empty((npar,), **f32) for _ in range(3))
        mt = torch.empty((S,), **f32)
        col = torch.empty((S,), **f32)
        pi = torch.empty((C, S), **f32)
        pibar = torch.empty((C, S), **f32)
        rowmax = torch.empty((C,), **f32)
        loss = torch.empty((), **f32)
        io = N.KbForwardIO(
            theta=N.ptr(theta), statewise=int(self.statewise), col_weights=N.ptr(col_weights),
            use_col_weights=int(use_col), e_init=float(so["e_init"]), e_max_iter=int(so["e_max_iter"]),
            e_tol=float(so["e_tol"]), pi_iters=int(so["pi_iters"]),
            E=N.ptr(E), E_s1=N.ptr(E_s1), E_s2=N.ptr(E_s2), Ebar=N.ptr(Ebar),
            log_pS=N.ptr(pS), log_pD=N.ptr(pD), log_pL=N.ptr(pL), max_coupling=N.ptr(mt),
            col_log_probs=N.ptr(col), pi=N.ptr(pi), pibar=N.ptr(pibar), pibar_row_max=N.ptr(rowmax),
            loss=N.ptr(loss),
        )
        if not self.statewise:
            pS, pD, pL = (t.reshape(()) for t in (pS, pD, pL))
        saved = dict(zip(FORWARD_SAVED_NAMES, (
            E, E_s1, E_s2, Ebar, pi.index_select(0, self.root_row_ids), pi, pibar, rowmax,
            pS, pD, pL, mt, col,
        )))
        saved["_use_col_weights"] = use_col
        return io, loss, saved, (theta, col_weights)

    def profile(self, enable: bool = True) -> None:
        """Record HIP events around every wave-kernel launch of later passes.

        While it is on, ``solve`` runs the forward and the backward one after the other
        (one launch per level and pass, on the caller's stream).
        """
        N.check(N.lib().kb_profile_enable(self._plan, int(bool(enable))))

    def level_launch_ms(self, which: str):
        """Per-level launch durations (ms) of the last forward / backward pass (``profile`` on).

        Index d is dependency level d (the backward runs the levels in reverse).
        """
        out = (ct.c_float * self.n_levels)()
        N.check(N.lib().kb_profile_read(self._plan, 0 if which == "forward" else 1, out, self.n_levels))
        return np.asarray(out[:], dtype=np.float64)

    def level_of_rows(self):
        """Clade-DAG depth of every row: 0 without splits, else 1 + max over its children."""
        a = self._arrays
        depth = np.zeros(self.C, dtype=np.int64)
        par, l, r = a["split_parent"], a["split_left"], a["split_right"]
        order = np.argsort(par, kind="stable")
        for i in order:  # parents in increasing row order; children precede parents
            d = 1 + max(depth[l[i]], depth[r[i]])
            if d > depth[par[i]]:
                depth[par[i]] = d
        return depth

    def level_shapes(self):
        """(rows, splits) of every dependency level."""
        depth = self.level_of_rows()
        rows = np.bincount(depth, minlength=self.n_levels)
        par = self._arrays["split_parent"]
        splits = np.bincount(depth[par], minlength=self.n_levels) if par.size else np.zeros_like(rows)
        return rows.astype(np.int64), splits.astype(np.int64)

    def forward_stats(self):
        n = ct.c_int32()
        l64 = ct.c_double()
        with torch.cuda.device(self.device):
            N.check(N.lib().kb_forward_stats(self._plan, ct.byref(n), ct.byref(l64), N.stream_handle(self.device)))
        self.last_n_e_iter = int(n.value)
        return {"n_e_iter": int(n.value), "loss64": float(l64.value)}

    def run_backward(self, theta, col_weights, saved, *, return_info=False, check_solve=True):
        """(forward intermediates) -> (grad_theta, grad_col), the reference ``run_backward`` contract.

        As in the reference (_implicit_grad.py:94), a failed E-adjoint BiCGSTAB
        solve raises ``RuntimeError``; checking it reads two status words back
        from the device once per backward (``check_solve=False`` skips the read,
        and ``backward_stats`` reports the status later).
        """
        io, grad_theta, grad_col, info = self._backward_args(theta, col_weights, saved, return_info)
        io.forward_token = self._token_of(saved)
        with torch.cuda.device(self.device):
            N.check(N.lib().kb_backward(self._plan, ct.byref(io), N.stream_handle(self.device)))
            if check_solve:
                self.backward_stats()
        if return_info:
            # neumann_terms: J^T applications of every solved row (255: not solved here)
            return grad_theta, grad_col, info
        return grad_theta, grad_col

    def _token_of(self, saved):
        last = self._last_forward
        if last is not None and last[1].matches(saved["pi_wave"]) and last[2].matches(saved["pibar_wave"]):
            return last[0]
        return 0

    def solve(self, theta, col_weights, *, use_col_weights=None, return_info=False, check_solve=True):
        """One forward and its backward -> (loss, saved, grad_theta, grad_col[, info]) (``kb_solve``).

        The values of ``run_forward`` followed by ``run_backward`` on its outputs; with a plan
        built under ``KB_OVERLAP_CUT`` the backward's rows of the families that end at or below
        that dependency level run on a second stream beside the forward's later levels.
        """
        fio, loss, saved, keep = self._forward_args(theta, col_weights, use_col_weights)
        bio, grad_theta, grad_col, info = self._backward_args(theta, col_weights, saved, return_info)
        self._keep_solve = keep
        with torch.cuda.device(self.device):
            N.check(N.lib().kb_solve(self._plan, ct.byref(fio), ct.byref(bio), N.stream_handle(self.device)))
            self._forward_done(saved)
            if check_solve:
                self.backward_stats()
        if return_info:
            return loss, saved, grad_theta, grad_col, info
        return loss, saved, grad_theta, grad_col

    def _backward_args(self, theta, col_weights, saved, return_info):
        """(kb_backward_io without its forward token, grad_theta, grad_col, info) of one backward."""
        lib = N.lib()
        if not hasattr(lib, "kb_backward"):
            raise N.NativeLibraryMissing("libkbench_hip was built without kb_backward")
        so = self.so
        if str(so["self_loop_solver"]).strip().lower() != "neumann":
            raise NotImplementedError("the fused backward implements the neumann self-loop solver")
        if float(so["pibar_side_threshold"]) != 0.0:
            # the row kernel skips only all-zero Pibar sides (the reference's rule at threshold 0)
            raise NotImplementedError("the fused backward implements pibar_side_threshold == 0 only")
        dev = self.device
        S, C = self.S, self.C
        theta_d = theta.detach().to(device=dev, dtype=torch.float32).contiguous()
        use_col = saved.get("_use_col_weights")
        use_col = self._use_col(col_weights) if use_col is None else bool(use_col)
        cw = col_weights.detach().to(device=dev, dtype=torch.float32).contiguous()
        f32 = dict(device=dev, dtype=torch.float32)
        grad_theta = torch.empty(tuple(theta_d.shape), **f32)
        grad_col = torch.empty((S,), **f32)
        mask = torch.empty((C,), device=dev, dtype=torch.uint8)
        acc = torch.empty((8, S), device=dev, dtype=torch.float64) if return_info else None
        terms = torch.full((C,), 255, device=dev, dtype=torch.uint8) if return_info else None
        c = lambda name: saved[name].detach().to(device=dev, dtype=torch.float32).contiguous()
        tens = {k: c(k) for k in ("E", "E_s1", "E_s2", "Ebar", "log_pS", "log_pD", "log_pL", "max_coupling",
                                  "col_log_probs", "pi_wave", "pibar_wave", "pibar_row_max")}
        io = N.KbBackwardIO(
            theta=N.ptr(theta_d), statewise=int(self.statewise), col_weights=N.ptr(cw), use_col_weights=int(use_col),
            neumann_terms=int(so["neumann_terms"]), pruning_threshold=float(so["adjoint_pruning_threshold"]),
            use_pruning=int(bool(so["use_adjoint_pruning"])), bicgstab_max_iter=int(so["bicgstab_max_iter"]),
            bicgstab_tol=float(so["bicgstab_tol"]), bicgstab_breakdown_tol=float(so["bicgstab_breakdown_tol"]),
            E=N.ptr(tens["E"]), E_s1=N.ptr(tens["E_s1"]), E_s2=N.ptr(tens["E_s2"]), Ebar=N.ptr(tens["Ebar"]),
            log_pS=N.ptr(tens["log_pS"]), log_pD=N.ptr(tens["log_pD"]), log_pL=N.ptr(tens["log_pL"]),
            max_coupling=N.ptr(tens["max_coupling"]), col_log_probs=N.ptr(tens["col_log_probs"]),
            pi=N.ptr(tens["pi_wave"]), pibar=N.ptr(tens["pibar_wave"]), pibar_row_max=N.ptr(tens["pibar_row_max"]),
            grad_theta=N.ptr(grad_theta), grad_col=N.ptr(grad_col), active_mask=N.ptr(mask), acc_out=N.ptr(acc),
            neumann_rtol=self.neumann_rtol, neumann_terms_out=N.ptr(terms),
        )
        self._keep = (tens, theta_d, cw)
        info = {"active_mask": mask, "acc": acc, "neumann_terms": terms} if return_info else None
        return io, grad_theta, grad_col, info

    def e_adjoint(self, saved, acc, *, q_extra=None, with_norm=False, use_col_weights=False, check_solve=True):
        """The E adjoint for the cotangents ``acc`` -> (w [S], g [5, S]), float64 (``kb_e_adjoint``).

        Solves (I - J_E^T) w = q at the saved E fixed point, q = acc_E + the (E_s1,
        E_s2, Ebar) cotangents pulled back to E + ``q_extra`` (+ the loss normaliser's
        E gradient with ``with_norm``); g holds the per-state cotangents of (log_pS,
        log_pD, log_pL, max_coupling, col_log_probs) of one E step at (w, acc_Ebar),
        plus acc's pS, pD, mt and col rows.  ``acc``: [8, S] (pD, pS, E, Ebar, E_s1,
        E_s2, max_coupling, col).  A failed BiCGSTAB raises ``RuntimeError`` (one
        status read, skipped with ``check_solve=False``: ``last_e_status`` then holds the
        device status words [iterations, failed] once the launch has run).
        """
        lib = N.lib()
        if not hasattr(lib, "kb_e_adjoint"):
            raise N.NativeLibraryMissing("libkbench_hip was built without kb_e_adjoint")
        so, dev, S = self.so, self.device, self.S
        f64 = dict(device=dev, dtype=torch.float64)
        acc = acc.detach().to(**f64).contiguous()
        if tuple(acc.shape) != (8, S):
            raise ValueError(f"acc must be [8, {S}]")
        qx = None if q_extra is None else q_extra.detach().to(**f64).reshape(S).contiguous()
        c = lambda name: saved[name].detach().to(device=dev, dtype=torch.float32).contiguous()
        tens = {k: c(k) for k in ("E", "log_pS", "log_pD", "log_pL", "max_coupling", "col_log_probs")}
        if int(tens["E"].numel()) != S:
            raise NotImplementedError("kb_e_adjoint solves one item row (itemwise=False)")
        w = torch.empty((S,), **f64)
        g = torch.empty((5, S), **f64)
        work = torch.empty((N.E_ADJOINT_WORK_VECTORS * S,), **f64)
        status = torch.zeros((2,), device=dev, dtype=torch.int32)
        io = N.KbEAdjointIO(
            statewise=int(self.statewise), use_col_weights=int(bool(use_col_weights)), with_norm=int(bool(with_norm)),
            bicgstab_max_iter=int(so["bicgstab_max_iter"]), bicgstab_tol=float(so["bicgstab_tol"]),
            bicgstab_breakdown_tol=float(so["bicgstab_breakdown_tol"]),
            E=N.ptr(tens["E"]), log_pS=N.ptr(tens["log_pS"]), log_pD=N.ptr(tens["log_pD"]),
            log_pL=N.ptr(tens["log_pL"]), max_coupling=N.ptr(tens["max_coupling"]),
            col_log_probs=N.ptr(tens["col_log_probs"]), acc=N.ptr(acc), q_extra=N.ptr(qx), w_out=N.ptr(w),
            g_out=N.ptr(g), work=N.ptr(work), status=N.ptr(status))
        with torch.cuda.device(dev):
            N.check(lib.kb_e_adjoint(self._plan, ct.byref(io), N.stream_handle(dev)))
        self._keep_e = (tens, acc, qx, work)
        self.last_e_status = status  # [iterations, failed] of this solve, once it has run
        if check_solve:
            it, failed = (int(x) for x in status.cpu())
            if failed:
                raise RuntimeError(f"E-adjoint BiCGSTAB solve failed after {it} iterations")
        return w, g

    def backward_stats(self):
        n = ct.c_int32()
        with torch.cuda.device(self.device):
            N.check(N.lib().kb_backward_stats(self._plan, ct.byref(n), N.stream_handle(self.device)))
        self.last_n_bicgstab = int(n.value)
        return {"n_bicgstab": int(n.value)}


def static_from_problem(problem: dict, device) -> SimpleNamespace:
    """Torch ``static`` namespace (the reference ``make_static`` result) from a generated problem."""
    from .runtime import make_static

    return make_static(problem_to_captured(problem), device)


def problem_to_captured(problem: dict) -> dict:
    """Generated numpy problem -> the reference's captured-dict format with torch tensors."""

    def conv(x):
        if isinstance(x, np.ndarray):
            if x.dtype == np.float64:
                return torch.from_numpy(x.astype(np.float32))
            return torch.from_numpy(x)
        if isinstance(x, dict):
            return {k: conv(v) for k, v in x.items()}
        if isinstance(x, list):
            return [conv(v) for v in x]
        return x

    st = problem["static"]
    return {
        "meta": dict(problem["meta"]),
        "static": {
            "wave_layout": conv(st["wave_layout"]),
            "state_helpers": conv(st["state_helpers"]),
            "rate_item_idx": conv(st["rate_item_idx"]),
            "itemwise": st["itemwise"],
            "statewise": st["statewise"],
        },
        "inputs": {k: conv(v) for k, v in problem["inputs"].items()},
    }
