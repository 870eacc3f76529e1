"""Backward wrappers on the HIP kernels (drop-in for the reference kbench/core/kernels/wave_backward.py).

Public functions (same names, signatures, return tuples and in-place
semantics as the reference):

* ``active_mask_from_rhs_absmax_fused`` (pristine wave_backward.py:168-201);
* ``wave_backward_uniform_fused`` (1398-1522 -> 969-1395): the self-loop
  adjoint and the per-element parameter contributions of one wave;
* ``dts_cross_backward_accum_fused`` (1980-2190): the split adjoint into the
  children's adjoint rows, parameter / coupling gradients and the staged Pibar
  cotangents u_d;
* ``uniform_cross_pibar_vjp_tree_from_ud_fused`` (2330-2446): the Pibar VJP
  of the staged u_d through the subtree sums.

Every cross-row accumulation (into ``accumulated_rhs``, ``grad_log_pD/pS``,
``grad_mt``, ``grad_col_log_probs``) is a fixed-order sum of per-split or
per-row contribution rows (``kb_rows_scatter_add`` / ``kb_rows_sum_into``)
instead of the reference's ``tl.atomic_add``, so repeated calls give
bitwise-identical gradients.

Self-loop solvers: ``"neumann"`` (the truncated series, one launch) and
``"gmres"`` (fixed-iteration GMRES over the whole wave, pristine
wave_backward.py:574-653: the Krylov loop runs on the host side in torch, each
operator application is one launch of the HIP kernel as one fixed-point step
from the basis vector with a zero right-hand side, which gives J^T x).
``self_loop_grad_targets`` adds the wave's bucket sums into the caller's
gradient accumulators (fixed-order row sums) instead of returning the bucket
rows (pristine wave_backward.py:1300-1395).
"""

from __future__ import annotations

import torch

from ..memory_policy import proposal0_memory_gate
from . import _hip as H
from ._dts_layout_contract import dts_backward_param_layout

__all__ = [
    "active_mask_from_rhs_absmax_fused",
    "wave_backward_uniform_fused",
    "dts_cross_backward_accum_fused",
    "uniform_cross_pibar_vjp_tree_from_ud_fused",
]

_SUPPORTED_FLOAT_DTYPES = (torch.float32, torch.float64, torch.bfloat16)


# ------------------------------------------------------------------ layouts
def _device_scalar_param(param, *, device, dtype):
    """One-element device tensor (reference wave_backward.py:23-31)."""
    if torch.is_tensor(param):
        if param.numel() != 1:
            raise ValueError("fused DTS backward scalar parameters must have one element")
        return param.to(device=device, dtype=dtype).reshape(1).contiguous()
    return torch.tensor([param], device=device, dtype=dtype)


def _dts_layout_param_args(log_pD, log_pS, *, item_idx, S, device, dtype):
    """(pD, pS, layout code) for the split backward (reference wave_backward.py:34-97).

    Codes: 0 shared scalar [1], 1 shared state vector [S], 2 item scalar [G]
    (by the parent's item), 3 item state [G, S].
    """

    def norm(param):
        if not torch.is_tensor(param):
            return _device_scalar_param(param, device=device, dtype=dtype), 0
        param = param.to(device=device, dtype=dtype)
        try:
            code = int(dts_backward_param_layout(param, S=S, item_indexed=item_idx is not None).code)
        except ValueError as exc:
            raise ValueError("DTS parameters must be scalar, [S], [G], [G, 1], or [G, S] "
                             "for the fused DTS backward path") from exc
        if code == 0:
            return param.reshape(1).contiguous(), 0
        if code == 2:
            return param.reshape(int(param.shape[0])).contiguous(), 2
        return param.contiguous(), code

    pD, lD = norm(log_pD)
    pS, lS = norm(log_pS)
    if lD != lS:
        raise ValueError("log_pD/log_pS must use the same DTS parameter layout")
    return pD, pS, lD


def _dts_grad_layout(grad, *, item_idx, S):
    try:
        return int(dts_backward_param_layout(grad, S=S, item_indexed=item_idx is not None).code)
    except ValueError as exc:
        raise ValueError("unsupported DTS gradient layout") from exc


def _uniform_backward_const_layout(const_tensor, item_idx, item_indexed):
    """0 shared [S], 1 row-expanded [W, S], 2 item-indexed [G, S] (reference wave_backward.py:100-117)."""
    if item_indexed:
        if item_idx is None:
            raise ValueError("item-indexed backward constants require item_idx")
        if const_tensor.ndim != 2:
            raise ValueError("item-indexed backward constants require [G, S] tensors")
        return 2
    return 1 if const_tensor.ndim == 2 else 0


def _uniform_backward_leaf_logp_mode(use_leaf_index, leaf_logp, item_idx, item_indexed):
    """Leaf log-probability addressing (reference wave_backward.py:120-135)."""
    if not use_leaf_index:
        return 0
    if item_indexed:
        if item_idx is None:
            raise ValueError("item-indexed leaf log-probabilities require item_idx")
        if leaf_logp.ndim == 1:
            return 1
        if leaf_logp.ndim == 2:
            if int(leaf_logp.shape[1]) == 1:
                raise ValueError("item-indexed [G, 1] leaf_logp should be expanded to [G, S]")
            return 2
        raise ValueError("item-indexed leaf_logp must have shape [G] or [G, S]")
    if leaf_logp.numel() == 1:
        return 3
    return 0


# ------------------------------------------------------------------ active mask
def active_mask_from_rhs_absmax_fused(rhs, threshold, *, use_pruning=True):
    """bool [W]: max_s |rhs[w, s]| >= threshold (> when pruning is off) (reference wave_backward.py:168-201)."""
    if rhs.ndim != 2:
        raise ValueError("rhs must be a 2D tensor")
    if rhs.device.type != "cuda":
        raise ValueError("active_mask_from_rhs_absmax_fused requires a CUDA tensor")
    if rhs.dtype not in _SUPPORTED_FLOAT_DTYPES:
        raise ValueError("active_mask_from_rhs_absmax_fused supports fp32/fp64/bf16 tensors")
    W, S = int(rhs.shape[0]), int(rhs.shape[1])
    active = torch.empty((W,), device=rhs.device, dtype=torch.bool)
    if W == 0:
        return active
    if S > 0 and rhs.stride(1) != 1:
        rhs = rhs.contiguous()
    code = {torch.float32: H.KB_F32, torch.float64: H.KB_F64, torch.bfloat16: H.KB_BF16}[rhs.dtype]
    H.check(H.lib().kb_active_mask(code, W, S, int(rhs.stride(0)) if S > 0 else 0, H.ptr(rhs), float(threshold),
                                   int(not use_pruning), H.ptr(active), H.stream(rhs.device)))
    return active


# ------------------------------------------------------------------ self-loop adjoint
def wave_backward_uniform_fused(Pi_star, Pibar_star, ws, W, S, dts_r, rhs, mt_squeezed, DL_const, Ebar, E, SL1_const,
                                SL2_const, col_log_probs, node_child1, node_child2, leaf_term_wt, neumann_terms=3,
                                leaf_state_idx=None, leaf_logp=None, has_leaf_term=True, active_mask=None,
                                node_parent=None, max_ancestor_depth=None, pibar_row_max=None, item_idx=None,
                                item_indexed_consts=False, compact_level_ptr=None, compact_level_parents=None,
                                compact_level_child1=None, compact_level_child2=None, grad_col_log_probs=None,
                                use_col_weights=True, self_loop_grad_targets=None, initial_v=None,
                                self_loop_solver="neumann", return_last_increment=False):
    """Self-loop adjoint of wave rows [ws, ws + W) (reference wave_backward.py:1398-1522).

    Returns ``(v_k, aw0, aw1, aw2, aw345, aw3, aw4)`` ([W, S] each; inactive
    rows zero), plus the per-row last-increment ratio with
    ``return_last_increment``.  ``grad_col_log_probs`` [S] is accumulated in
    place.
    """
    W, S, ws = int(W), int(S), int(ws)
    use_leaf_index = bool(has_leaf_term) and leaf_state_idx is not None and leaf_logp is not None
    const_layout = _uniform_backward_const_layout(DL_const, item_idx, bool(item_indexed_consts))
    if bool(item_indexed_consts) and use_leaf_index:
        if leaf_logp.ndim == 1:
            leaf_logp = leaf_logp.unsqueeze(-1).expand(-1, S).contiguous()
        elif leaf_logp.ndim == 2 and int(leaf_logp.shape[1]) == 1:
            leaf_logp = leaf_logp.expand(-1, S).contiguous()
    leaf_mode = _uniform_backward_leaf_logp_mode(use_leaf_index, leaf_logp, item_idx, bool(item_indexed_consts))
    if node_parent is None:
        raise ValueError("node_parent is required for the retained backward fast path")
    if max_ancestor_depth is None:
        raise ValueError("max_ancestor_depth is required for the retained backward fast path")
    if pibar_row_max is None:
        raise ValueError("pibar_row_max is required for the retained backward fast path")
    if Pi_star.device.type != "cuda":
        raise RuntimeError("the self-loop backward requires HIP device tensors")
    if Pi_star.dtype not in (torch.float32, torch.float64):
        raise RuntimeError("the self-loop backward supports fp32/fp64 only")
    if any(t is None for t in (compact_level_ptr, compact_level_parents, compact_level_child1, compact_level_child2)):
        raise ValueError("compact state levels are required for the retained 2D self-loop path")
    solver = str(self_loop_solver).strip().lower()
    if solver not in ("neumann", "gmres"):
        raise ValueError(f"unsupported self-loop solver {self_loop_solver!r}")
    if solver == "gmres" and initial_v is not None:
        raise ValueError("GMRES self-loop solve does not support initial_v")
    if self_loop_grad_targets is not None and len(self_loop_grad_targets) != 8:
        raise ValueError("self_loop_grad_targets must hold grad_log_pD, grad_log_pS, grad_E, grad_Ebar, grad_E_s1, "
                         "grad_E_s2, grad_mt and param_grad_vector")
    ok, need, budget = proposal0_memory_gate(W, S, Pi_star.dtype, device=Pi_star.device)
    if not ok:
        raise RuntimeError(f"2D self-loop fast path estimated scratch {need / 1024 ** 3:.2f} GiB above memory "
                           f"budget {(budget or 0) / 1024 ** 3:.2f} GiB")
    dt, dev = Pi_star.dtype, Pi_star.device
    outs = [torch.empty((W, S), device=dev, dtype=dt) for _ in range(7)]
    if W == 0:
        return (*outs, None) if return_last_increment else tuple(outs)
    if not Pi_star.is_contiguous() or not Pibar_star.is_contiguous():
        raise ValueError("Pi_star and Pibar_star must be contiguous [C, S] tensors")
    tree = H.tree_from_parent(node_parent, node_child1, node_child2)
    consts = [H.f(c, dt, dev) for c in (mt_squeezed, DL_const, Ebar, E, SL1_const, SL2_const)]
    if const_layout == 0:
        consts = [c.reshape(-1) for c in consts]
    col = H.f(col_log_probs, dt, dev)
    rmax = H.f(pibar_row_max, dt, dev)
    rhs_c = H.f(rhs, dt, dev)
    dts = H.f(dts_r, dt, dev)
    v0 = None
    if initial_v is not None:
        if tuple(initial_v.shape) != (W, S):
            raise ValueError(f"initial_v shape {tuple(initial_v.shape)} does not match wave scratch shape {(W, S)}")
        v0 = H.f(initial_v, dt, dev)
    act = None if active_mask is None else active_mask.to(device=dev, dtype=torch.bool).contiguous()
    item = H.i64(item_idx, dev)
    leaf = H.i64(leaf_state_idx, dev) if use_leaf_index else None
    lp = H.f(leaf_logp, dt, dev) if use_leaf_index else None
    lterm = H.f(leaf_term_wt, dt, dev) if (leaf_term_wt is not None and not use_leaf_index and has_leaf_term) else None
    col_rows = torch.empty((W, S), device=dev, dtype=dt)
    relres = (torch.empty((W,), device=dev, dtype=torch.float32)
              if return_last_increment and solver == "neumann" else None)

    def launch(rhs_t, v0_t, n_terms, out, col_out, relres_t):
        io = H.KbWaveBwdIO(
            dtype=H.dtype_code(dt), S=S, W=W, n_terms=int(n_terms), const_layout=const_layout, leaf_mode=leaf_mode,
            use_leaf_index=int(use_leaf_index), use_col_weights=int(bool(use_col_weights)), ws=ws,
            Pi=H.ptr(Pi_star), Pibar=H.ptr(Pibar_star), pibar_row_max=H.ptr(rmax), dts=H.ptr(dts), rhs=H.ptr(rhs_t),
            initial_v=H.ptr(v0_t), active=H.ptr(act), max_coupling=H.ptr(consts[0]), DL=H.ptr(consts[1]),
            Ebar=H.ptr(consts[2]), E=H.ptr(consts[3]), SL1=H.ptr(consts[4]), SL2=H.ptr(consts[5]),
            col_log_probs=H.ptr(col), item_idx=H.ptr(item), leaf_state=H.ptr(leaf), leaf_logp=H.ptr(lp),
            leaf_term=H.ptr(lterm), v=H.ptr(out[0]), aw0=H.ptr(out[1]), aw1=H.ptr(out[2]), aw2=H.ptr(out[3]),
            aw345=H.ptr(out[4]), aw3=H.ptr(out[5]), aw4=H.ptr(out[6]), col_rows=H.ptr(col_out),
            relres=H.ptr(relres_t),
        )
        H.check(H.lib().kb_wave_backward(tree.handle, io, H.stream(dev)))

    if solver == "neumann":
        launch(rhs_c, v0, neumann_terms, outs, col_rows, relres)
    else:
        # A x = x - J^T x on the active rows (the kernel zeroes inactive rows)
        zero = torch.zeros_like(rhs_c)
        scratch = [torch.empty((W, S), device=dev, dtype=dt) for _ in range(8)]

        def apply_a(x):
            launch(zero, x, 1, scratch, scratch[7], None)
            return x - scratch[0]

        g_rhs = rhs_c if act is None else rhs_c * act[:, None].to(dt)
        v_sol = _gmres_fixed(apply_a, g_rhs.contiguous(), int(neumann_terms))
        # outputs from the solution: no further step (n_terms = 0 keeps v = v_sol)
        launch(rhs_c, v_sol.contiguous(), 0, outs, col_rows, None)
    if grad_col_log_probs is not None:
        H.sum_rows_into(grad_col_log_probs, col_rows)
    if self_loop_grad_targets is not None:
        _accumulate_grad_targets(self_loop_grad_targets, outs, S)
        base = (outs[0], None, None, None, None, None, None)
    else:
        base = tuple(outs)
    if return_last_increment:
        last = relres if (solver == "neumann" and initial_v is None and int(neumann_terms) > 0) else None
        return (*base, last)
    return base


def _gmres_fixed(apply_a, b, max_iter):
    """Fixed-iteration unrestarted GMRES over the whole wave (pristine wave_backward.py:574-653).

    Classical Gram-Schmidt with one reorthogonalisation; stops early when the
    new basis norm falls to eps * max(|b|, 1); the (at most 17 x 16)
    Hessenberg least-squares problem is solved on the host in float64.
    """
    m = int(max_iter)
    if m < 1:
        return torch.zeros_like(b)
    b_norm = torch.linalg.vector_norm(b)
    bn = float(b_norm)
    if bn == 0.0:
        return torch.zeros_like(b)
    flat = b.reshape(-1)
    Q = torch.empty((m + 1, flat.numel()), dtype=b.dtype, device=b.device)
    Hs = torch.zeros((m + 1, m), dtype=b.dtype, device=b.device)
    Q[0] = flat / b_norm
    tol = torch.finfo(b.dtype).eps * max(bn, 1.0)
    tiny = torch.finfo(b.dtype).tiny
    k = m
    for j in range(m):
        w = apply_a(Q[j].view_as(b)).reshape(-1)
        q = Q[: j + 1]
        c = torch.mv(q, w)
        w = torch.addmv(w, q.t(), c, alpha=-1.0)
        c2 = torch.mv(q, w)
        w = torch.addmv(w, q.t(), c2, alpha=-1.0)
        Hs[: j + 1, j] = c + c2
        h = torch.linalg.vector_norm(w)
        Hs[j + 1, j] = h
        if float(h) <= tol:
            k = j + 1
            break
        if j + 1 < m:
            Q[j + 1] = w / torch.clamp(h, min=tiny)
    Hh = Hs[: k + 1, :k].double().cpu()
    e1 = torch.zeros((k + 1,), dtype=torch.float64)
    e1[0] = bn
    y = torch.linalg.lstsq(Hh, e1.unsqueeze(-1)).solution.squeeze(-1)
    return torch.mv(Q[:k].t(), y.to(device=b.device, dtype=b.dtype)).view_as(b)


def _accumulate_grad_targets(targets, outs, S):
    """Add the wave's bucket sums over rows into the caller's accumulators (pristine wave_backward.py:906-953).

    Per state s: grad_E += aw0 + aw2, grad_Ebar += aw1, grad_E_s1 += aw4,
    grad_E_s2 += aw3, grad_mt += aw2; grad_log_pD += aw0 and grad_log_pS +=
    aw345 per state with ``param_grad_vector``, else summed over states into
    their first element.  Accumulators are addressed by state (their first S
    elements), as the reference's pointer arithmetic does.
    """
    gpD, gpS, gE, gEbar, gEs1, gEs2, gmt, vec = targets
    _v, aw0, aw1, aw2, aw345, aw3, aw4 = outs

    def add_states(dst, src):
        if dst is None:
            return
        flat = dst.reshape(-1)
        if flat.numel() < S:
            raise ValueError("self-loop gradient targets need at least S elements")
        view = flat[:S]
        if view.dtype == src.dtype and view.is_contiguous():
            H.sum_rows_into(view, src)
        else:
            tmp = torch.zeros((S,), device=src.device, dtype=src.dtype)
            H.sum_rows_into(tmp, src)
            view.add_(tmp.to(view.dtype))

    def add_scalar(dst, src):
        if dst is None:
            return
        tmp = torch.zeros((S,), device=src.device, dtype=src.dtype)
        H.sum_rows_into(tmp, src)
        tot = torch.zeros((1,), device=src.device, dtype=src.dtype)
        H.sum_rows_into(tot, tmp.reshape(S, 1))
        dst.reshape(-1)[:1].add_(tot.to(dst.dtype))

    add_states(gE, aw0)
    add_states(gE, aw2)
    add_states(gEbar, aw1)
    add_states(gEs1, aw4)
    add_states(gEs2, aw3)
    add_states(gmt, aw2)
    if bool(vec):
        add_states(gpD, aw0)
        add_states(gpS, aw345)
    else:
        add_scalar(gpD, aw0)
        add_scalar(gpS, aw345)


# ------------------------------------------------------------------ split adjoint
def dts_cross_backward_accum_fused(Pi_star, Pibar_star, v_k, ws, sl, sr, reduce_idx, wlsp, log_pD, log_pS,
                                   node_child1, node_child2, accumulated_rhs, S, active_mask=None, use_atomics=True,
                                   merge_s_term=False, grad_log_pD=None, grad_log_pS=None, grad_mt=None,
                                   accum_param_reductions=False, accum_mt_reduction=False, output_pibar_ud=False,
                                   output_pibar_side_active=False, pibar_side_threshold=0.0, mt_squeezed=None,
                                   pibar_row_max=None, grad_mt_two_stage=False, grad_mt_two_stage_tile_splits=128,
                                   skip_inactive_pibar_output_zero=False, item_idx=None):
    """Split adjoint of one wave (reference wave_backward.py:1980-2190).

    ``accumulated_rhs`` [C, S] receives the children's direct Pi adjoints in
    place.  Returns ``(pibar_ud, pibar_A, pibar_side_active, param_pD,
    param_pS)`` with ``output_pibar_ud`` and ``output_pibar_side_active``,
    ``(pibar_ud, pibar_A, param_pD, param_pS)`` with ``output_pibar_ud`` only,
    else ``(grad_Pibar_l, grad_Pibar_r, param_pD, param_pS)``; ``param_pD`` /
    ``param_pS`` are None when ``accum_param_reductions`` adds them into
    ``grad_log_pD`` / ``grad_log_pS``.  ``use_atomics``, ``merge_s_term`` and the
    ``grad_mt_two_stage*`` options select reference launch variants with the
    same result and are accepted for compatibility.
    """
    S = int(S)
    n = int(sl.shape[0])
    dev, dt = Pi_star.device, Pi_star.dtype
    H.require_device(Pi_star, "dts_cross_backward_accum_fused")
    H.dtype_code(dt)
    item = H.i64(item_idx, dev)
    pD, pS, player = _dts_layout_param_args(log_pD, log_pS, item_idx=item, S=S, device=dev, dtype=dt)
    if accum_param_reductions and (grad_log_pD is None or grad_log_pS is None):
        raise ValueError("grad_log_pD/grad_log_pS are required when accumulating DTS scalar reductions")
    glayout = 0
    if accum_param_reductions:
        glayout = _dts_grad_layout(grad_log_pD, item_idx=item, S=S)
        if glayout != _dts_grad_layout(grad_log_pS, item_idx=item, S=S):
            raise ValueError("grad_log_pD/grad_log_pS must use the same DTS gradient layout")
    if accum_mt_reduction and grad_mt is None:
        raise ValueError("grad_mt is required when accumulating DTS mt reductions")
    gmt_layout = 0
    if accum_mt_reduction:
        if grad_mt.numel() == 1 or (grad_mt.ndim == 1 and int(grad_mt.shape[0]) == S):
            gmt_layout = 0
        elif item is not None and grad_mt.ndim == 2 and int(grad_mt.shape[1]) == S:
            gmt_layout = 1
        else:
            raise ValueError("DTS mt reduction target must be scalar, [S], or [G, S]")
    if output_pibar_ud and (mt_squeezed is None or pibar_row_max is None):
        raise ValueError("mt_squeezed and pibar_row_max are required when outputting Pibar u_d")
    mt_layout = 0
    if output_pibar_ud:
        if mt_squeezed.ndim == 1 and int(mt_squeezed.shape[0]) == S:
            mt_layout = 0
        elif item is not None and mt_squeezed.ndim == 2 and int(mt_squeezed.shape[1]) == S:
            mt_layout = 1
        else:
            raise ValueError("mt_squeezed must have shape [S] or [G, S] when outputting Pibar u_d")
        if pibar_row_max.numel() < Pi_star.shape[0]:
            raise ValueError("pibar_row_max must contain one row-max value per Pi row")
    if output_pibar_side_active and not output_pibar_ud:
        raise ValueError("output_pibar_side_active requires output_pibar_ud")
    if torch.is_tensor(pibar_side_threshold):
        if pibar_side_threshold.numel() != 1:
            raise ValueError("pibar_side_threshold tensor must contain one value")
        thr = float(pibar_side_threshold.detach().reshape(()).item())
    else:
        thr = float(pibar_side_threshold)
        if thr < 0.0:
            raise ValueError("pibar_side_threshold must be non-negative")
    side_thr = thr if output_pibar_side_active else 0.0

    ud = A = side_active = gPl = gPr = None
    if output_pibar_ud:
        ud = torch.empty((2 * n, S), device=dev, dtype=dt)
        A = torch.empty((2 * n,), device=dev, dtype=dt)
        if output_pibar_side_active:
            side_active = torch.empty((2 * n,), device=dev, dtype=torch.bool)
    else:
        gPl = torch.empty((n, S), device=dev, dtype=dt)
        gPr = torch.empty((n, S), device=dev, dtype=dt)
    param_pD = param_pS = None
    if n == 0:
        if not accum_param_reductions:
            param_pD = torch.empty((0,), device=dev, dtype=dt)
            param_pS = torch.empty((0,), device=dev, dtype=dt)
        return _cross_result(output_pibar_ud, output_pibar_side_active, ud, A, side_active, gPl, gPr,
                             param_pD, param_pS)
    # contribution rows, summed in a fixed order below
    side_rows = torch.empty((2 * n, S), device=dev, dtype=dt)
    need_rows = accum_param_reductions and glayout in (1, 3)
    need_sums = (not accum_param_reductions) or glayout in (0, 2)
    param_rows = torch.empty((2 * n, S), device=dev, dtype=dt) if need_rows else None
    param_sums = torch.empty((2 * n,), device=dev, dtype=dt) if need_sums else None
    mt_rows = torch.empty((2 * n, S), device=dev, dtype=dt) if accum_mt_reduction else None
    sl64, sr64, red = H.i64(sl, dev), H.i64(sr, dev), H.i64(reduce_idx, dev)
    act = None if active_mask is None else active_mask.to(device=dev, dtype=torch.bool).contiguous()
    wl = H.f(wlsp.squeeze(-1) if wlsp.ndim > 1 else wlsp, dt, dev)
    mt = H.f(mt_squeezed, dt, dev) if output_pibar_ud else None
    rmax = H.f(pibar_row_max, dt, dev) if output_pibar_ud else None
    vk = H.f(v_k, dt, dev)
    c1, c2 = H.i64(node_child1, dev), H.i64(node_child2, dev)
    io = H.KbDtsCrossIO(
        dtype=H.dtype_code(dt), S=S, param_layout=player, mt_layout=mt_layout, output_ud=int(bool(output_pibar_ud)),
        skip_inactive_ud_zero=int(bool(skip_inactive_pibar_output_zero)), N=n, ws=int(ws), side_threshold=side_thr,
        node_child1=H.ptr(c1), node_child2=H.ptr(c2), Pi=H.ptr(Pi_star), Pibar=H.ptr(Pibar_star), v=H.ptr(vk),
        active=H.ptr(act), sl=H.ptr(sl64), sr=H.ptr(sr64), reduce_idx=H.ptr(red), wlsp=H.ptr(wl), log_pD=H.ptr(pD),
        log_pS=H.ptr(pS), item_idx=H.ptr(item), mt=H.ptr(mt), pibar_row_max=H.ptr(rmax),
        side_rows=H.ptr(side_rows), ud=H.ptr(ud), A=H.ptr(A), side_active=H.ptr(side_active),
        grad_Pibar_l=H.ptr(gPl), grad_Pibar_r=H.ptr(gPr), param_rows=H.ptr(param_rows),
        param_sums=H.ptr(param_sums), mt_rows=H.ptr(mt_rows),
    )
    H.check(H.lib().kb_dts_cross_backward(io, H.stream(dev)))

    # children's adjoint rows: side r of split i goes to row sl[i] (r < n) or sr[i]
    H.scatter_add_rows(accumulated_rhs, side_rows, lambda: torch.cat((sl64, sr64)), static=(sl64, sr64))
    sums = []  # (accumulator row, contribution rows): one fixed-order launch for all of them
    if accum_param_reductions:
        if glayout == 1 or (glayout == 3 and int(grad_log_pD.shape[0]) == 1):
            # one parameter row: every split adds into it (parallel fixed-order row sum)
            sums += [(grad_log_pD.reshape(-1), param_rows[:n]), (grad_log_pS.reshape(-1), param_rows[n:])]
        elif glayout == 0:
            H.sum_rows_into(grad_log_pD.reshape(-1), param_sums[:n].reshape(n, 1))
            H.sum_rows_into(grad_log_pS.reshape(-1), param_sums[n:].reshape(n, 1))
        else:
            if item is None:
                raise ValueError("per-item parameter gradients need item_idx")
            st = (item, red, int(ws))
            pkey = lambda: item.index_select(0, red + int(ws))
            if glayout == 3:
                H.scatter_add_rows(grad_log_pD.reshape(-1), param_rows[:n], pkey, row_stride=S, static=st)
                H.scatter_add_rows(grad_log_pS.reshape(-1), param_rows[n:], pkey, row_stride=S, static=st)
            else:
                H.scatter_add_rows(grad_log_pD.reshape(-1), param_sums[:n].reshape(n, 1), pkey, row_stride=1,
                                   static=st)
                H.scatter_add_rows(grad_log_pS.reshape(-1), param_sums[n:].reshape(n, 1), pkey, row_stride=1,
                                   static=st)
    else:
        param_pD, param_pS = param_sums[:n].clone(), param_sums[n:].clone()
    if accum_mt_reduction:
        if gmt_layout == 1 and int(grad_mt.shape[0]) == 1:
            sums.append((grad_mt.reshape(-1), mt_rows))
        elif gmt_layout == 1:
            H.scatter_add_rows(grad_mt.reshape(-1), mt_rows,
                               lambda: torch.cat((item.index_select(0, sl64), item.index_select(0, sr64))),
                               row_stride=S, static=(item, sl64, sr64))
        elif grad_mt.numel() == 1:
            tmp = torch.zeros((S,), device=dev, dtype=dt)
            H.sum_rows_into(tmp, mt_rows)
            H.sum_rows_into(grad_mt.reshape(1, 1), tmp.reshape(S, 1))
        else:
            H.sum_rows_into(grad_mt.reshape(-1), mt_rows)
    if len({int(d.data_ptr()) for d, _ in sums}) == len(sums):
        H.rows_sum_accum(sums)
    else:  # accumulators that share storage: one at a time
        for d, rows in sums:
            H.sum_rows_into(d, rows)
    return _cross_result(output_pibar_ud, output_pibar_side_active, ud, A, side_active, gPl, gPr, param_pD, param_pS)


def _cross_result(output_ud, output_side, ud, A, side_active, gPl, gPr, param_pD, param_pS):
    if output_ud:
        if output_side:
            return ud, A, side_active, param_pD, param_pS
        return ud, A, param_pD, param_pS
    return gPl, gPr, param_pD, param_pS


# ------------------------------------------------------------------ Pibar VJP
def uniform_cross_pibar_vjp_tree_from_ud_fused(Pi_star, col_log_probs, pibar_ud, pibar_A, sl, sr, accumulated_rhs, S,
                                               active_mask=None, reduce_idx=None, pibar_row_max=None,
                                               skip_zero_sides=False, side_active=None, compact_level_ptr=None,
                                               compact_level_parents=None, compact_level_child1=None,
                                               compact_level_child2=None, grad_col_log_probs=None,
                                               use_col_weights=True, side_active_threshold=0.0):
    """Pibar VJP of the staged u_d (reference wave_backward.py:2330-2446).

    For every split side that is active, ``pibar_ud`` row is replaced in
    place by its subtree sums and p'(child) * (A - subtree(u_d)) is added into
    ``accumulated_rhs[child]`` and ``grad_col_log_probs``.  Returns the side
    mask used (None when neither ``side_active`` nor ``skip_zero_sides``).
    """
    S = int(S)
    n = int(sl.shape[0])
    if n == 0:
        return None
    if active_mask is not None and reduce_idx is None:
        raise ValueError("reduce_idx is required when active_mask is provided")
    if pibar_row_max is None:
        raise ValueError("pibar_row_max is required for DTS-staged Pibar VJP")
    if torch.is_tensor(side_active_threshold):
        if side_active_threshold.numel() != 1:
            raise ValueError("side_active_threshold tensor must contain one value")
        thr = float(side_active_threshold.detach().reshape(()).item())
    else:
        thr = float(side_active_threshold)
        if thr < 0.0:
            raise ValueError("side_active_threshold must be non-negative")
    dev, dt = Pi_star.device, Pi_star.dtype
    H.require_device(Pi_star, "uniform_cross_pibar_vjp_tree_from_ud_fused")
    H.dtype_code(dt)
    if side_active is not None:
        if side_active.numel() != 2 * n:
            raise ValueError("side_active must have one entry per split side")
        side_active = side_active.to(device=dev, dtype=torch.bool).contiguous()
    elif skip_zero_sides:
        side_active = _side_active_from_ud(pibar_ud, thr)
    if any(t is None for t in (compact_level_ptr, compact_level_parents, compact_level_child1, compact_level_child2)):
        raise ValueError("compact state levels are required for Pibar VJP")
    if compact_level_ptr.numel() < 2:
        raise ValueError("compact_level_ptr must contain at least start and end offsets")
    if not pibar_ud.is_contiguous() or pibar_ud.dtype != dt:
        raise ValueError("pibar_ud must be a contiguous [2N, S] tensor of the Pi dtype")
    tree = H.tree_from_levels(S, compact_level_ptr, compact_level_parents, compact_level_child1,
                              compact_level_child2)
    sl64, sr64 = H.i64(sl, dev), H.i64(sr, dev)
    red = H.i64(reduce_idx, dev)
    act = None if active_mask is None else active_mask.to(device=dev, dtype=torch.bool).contiguous()
    col = H.f(col_log_probs, dt, dev)
    A = H.f(pibar_A, dt, dev)
    rmax = H.f(pibar_row_max, dt, dev)
    contrib = torch.empty((2 * n, S), device=dev, dtype=dt)
    io = H.KbPibarVjpIO(
        dtype=H.dtype_code(dt), S=S, use_col_weights=int(bool(use_col_weights)), N=n, Pi=H.ptr(Pi_star),
        col_log_probs=H.ptr(col), ud=H.ptr(pibar_ud), A=H.ptr(A), side_active=H.ptr(side_active), sl=H.ptr(sl64),
        sr=H.ptr(sr64), reduce_idx=H.ptr(red), active=H.ptr(act), pibar_row_max=H.ptr(rmax),
        contrib=H.ptr(contrib),
    )
    H.check(H.lib().kb_pibar_vjp(tree.handle, io, H.stream(dev)))
    H.wrote(pibar_ud)
    H.scatter_add_rows(accumulated_rhs, contrib, lambda: torch.cat((sl64, sr64)), static=(sl64, sr64))
    if grad_col_log_probs is not None:
        H.sum_rows_into(grad_col_log_probs, contrib)
    return side_active


def _side_active_from_ud(pibar_ud, thr):
    """Sides whose staged u_d has any nonzero entry (abs-sum above thr when thr > 0)."""
    a = pibar_ud.abs()
    if thr > 0.0:
        return (a.sum(dim=1) > thr).contiguous()
    return (a.amax(dim=1) != 0).contiguous() if a.shape[1] else torch.zeros(a.shape[0], dtype=torch.bool,
                                                                            device=a.device)
