"""E-step wrappers on the HIP kernels (drop-in for the reference kbench/core/kernels/e_step.py).

* ``e_step_triton_autograd`` -- one E-step with a VJP, as a torch autograd
  function (reference e_step.py:290-435);
* ``e_fixed_point_triton`` -- the E fixed point (reference e_step.py:438-501).

The names are the reference's, so the glue imports them unchanged.  Both run
on ``kb_estep`` / ``kb_estep_vjp`` (include/kbench_ops.h), one workgroup per
item row, float64 arithmetic, no host synchronisation: the fixed point loops
on the device.  Differences from the reference, all inside its tolerances:
the iteration runs in float64 (the reference's stopping rule e_tol = 1e-8 is
below float32 resolution, so a float32 iterate can cycle at the last bit until
max_iter), and each item row stops on its own once its max |E_new - E| < tol
instead of all rows iterating until the largest difference is below tol.
"""

from __future__ import annotations

import torch

from ..parameters.extract_parameters import as_item_state
from . import _hip as H

__all__ = ["e_step_triton_autograd", "e_fixed_point_triton"]


def _estep(tree, E, pS, pD, pL, mt, col, use_col, *, mode, max_iter=1, tol=1.0, max_diff=None, n_iter=None):
    G, S = int(E.shape[0]), int(E.shape[1])
    outs = [torch.empty_like(E) for _ in range(4)]
    io = H.KbEStepIO(
        dtype=H.dtype_code(E.dtype), G=G, mode=int(mode), use_col_weights=int(bool(use_col)),
        max_iter=int(max_iter), tol=float(tol), E=H.ptr(E), log_pS=H.ptr(pS), log_pD=H.ptr(pD), log_pL=H.ptr(pL),
        max_coupling=H.ptr(mt), col_log_probs=H.ptr(col), E_out=H.ptr(outs[0]), E_s1=H.ptr(outs[1]),
        E_s2=H.ptr(outs[2]), Ebar=H.ptr(outs[3]), max_diff=H.ptr(max_diff), n_iter=H.ptr(n_iter),
    )
    H.check(H.lib().kb_estep(tree.handle, io, H.stream(E.device)))
    return tuple(outs)


def _prepare(E, params, col_log_probs):
    H.require_device(E, "the E-step")
    dt, dev = E.dtype, E.device
    H.dtype_code(dt)
    G, S = int(E.shape[0]), int(E.shape[1])
    mats = [H.f(as_item_state(p, S, G), dt, dev) for p in params]
    return mats, H.f(col_log_probs, dt, dev)


class _EStep(torch.autograd.Function):
    """One E-step; backward is the E-step VJP kernel (reference e_step.py:290-407)."""

    @staticmethod
    def forward(ctx, E, pS, pD, pL, mt, col, node_parent, node_child1, node_child2, max_ancestor_depth,
                use_col_weights):
        tree = H.tree_from_parent(node_parent, node_child1, node_child2)
        out = _estep(tree, E, pS, pD, pL, mt, col, use_col_weights, mode=0)
        ctx.save_for_backward(E, *out, pS, pD, pL, col)
        ctx.tree = tree
        ctx.use_col = bool(use_col_weights)
        return out

    @staticmethod
    def backward(ctx, gN, g1, g2, gB):
        E, En, Es1, Es2, Eb, pS, pD, pL, col = ctx.saved_tensors
        G, S = int(E.shape[0]), int(E.shape[1])
        gN, g1, g2, gB = (torch.zeros_like(E) if g is None else g.to(E.dtype).contiguous() for g in (gN, g1, g2, gB))
        gE, gpS, gpD, gpL, gmt = (torch.empty_like(E) for _ in range(5))
        gcol = torch.zeros_like(col)
        work = torch.empty((G, S), device=E.device, dtype=torch.float64)
        io = H.KbEStepVjpIO(
            dtype=H.dtype_code(E.dtype), G=G, use_col_weights=int(ctx.use_col),
            E=H.ptr(E), E_new=H.ptr(En), E_s1=H.ptr(Es1), E_s2=H.ptr(Es2), Ebar=H.ptr(Eb),
            log_pS=H.ptr(pS), log_pD=H.ptr(pD), log_pL=H.ptr(pL), col_log_probs=H.ptr(col),
            g_E_new=H.ptr(gN), g_E_s1=H.ptr(g1), g_E_s2=H.ptr(g2), g_Ebar=H.ptr(gB),
            grad_E=H.ptr(gE), grad_log_pS=H.ptr(gpS), grad_log_pD=H.ptr(gpD), grad_log_pL=H.ptr(gpL),
            grad_max_coupling=H.ptr(gmt), grad_col_log_probs=H.ptr(gcol), work=H.ptr(work),
        )
        H.check(H.lib().kb_estep_vjp(ctx.tree.handle, io, H.stream(E.device)))
        return gE, gpS, gpD, gpL, gmt, gcol, None, None, None, None, None


def e_step_triton_autograd(E, log_pS, log_pD, log_pL, max_coupling, col_log_probs, node_parent, node_child1,
                           node_child2, max_ancestor_depth, use_col_weights=True):
    """(E_new, E_s1, E_s2, Ebar) of one E-step, differentiable (reference e_step.py:410-435).

    Parameters of shape [S], [G, 1], scalar ... are expanded to [G, S] with
    ``as_item_state`` inside the autograd graph, so their gradients come back
    reduced to the caller's shapes.
    """
    E_arg = E.contiguous()
    G, S = int(E_arg.shape[0]), int(E_arg.shape[1])
    H.require_device(E_arg, "e_step_triton_autograd")
    H.dtype_code(E_arg.dtype)
    mats = [as_item_state(p, S, G).to(E_arg.dtype).contiguous() for p in (log_pS, log_pD, log_pL, max_coupling)]
    return _EStep.apply(E_arg, *mats, col_log_probs.to(E_arg.dtype).contiguous(), node_parent, node_child1,
                        node_child2, int(max_ancestor_depth), bool(use_col_weights))


def e_fixed_point_triton(E0, log_pS, log_pD, log_pL, max_coupling, col_log_probs, node_parent, node_child1,
                         node_child2, max_ancestor_depth, *, max_iter=2000, tol=1e-8, use_col_weights=True):
    """(E, E_s1, E_s2, Ebar) at the E fixed point (reference e_step.py:438-501)."""
    max_iter = int(max_iter)
    tol = float(tol)
    if max_iter < 1:
        raise ValueError("max_iter must be at least 1")
    if tol <= 0.0:
        raise ValueError("tol must be positive")
    E_a = E0.contiguous()
    mats, col = _prepare(E_a, (log_pS, log_pD, log_pL, max_coupling), col_log_probs)
    tree = H.tree_from_parent(node_parent, node_child1, node_child2)
    with torch.no_grad():
        return _estep(tree, E_a.detach(), *mats, col, use_col_weights, mode=1, max_iter=max_iter, tol=tol)
