"""Entry points with the reference's ``kbench.runtime`` contract, on the native whole-pass driver.

Contract (reference kbench/runtime.py:29-115):

* ``make_static(captured, device)`` -> the ``static`` namespace: ``wave_layout``,
  ``state_helpers``, ``rate_item_idx`` on ``device``, ``itemwise``,
  ``statewise``, a validated ``solver_options`` and ``warm_E`` (None);
* ``run_forward(static, theta, col_weights) -> (loss, saved)``, ``saved`` keyed
  by ``FORWARD_SAVED_NAMES``;
* ``run_backward(static, theta, col_weights, saved) -> (grad_theta, grad_col)``.

Here both passes run on ``kbench.fused.FusedSolver``: one plan of
device-resident layout tables per ``static`` (created on first use and kept
with it), then a few kernels per dependency level.  The reference's own Python
glue is not part of this package; its per-call wrappers (``kbench.core.kernels``)
are, for callers that drive them one call at a time.

Two backward options change what is computed per wave, and the whole-pass
driver does not implement them: ``self_loop_solver="gmres"`` (its Krylov space
spans a wave, so the result depends on the wave grouping, which the driver
replaces by dependency levels) and ``pibar_side_threshold > 0`` (split sides
whose staged Pibar adjoint has a small abs-sum are dropped).  With either set,
``run_backward`` runs the per-call drivers of ``kbench.percall`` instead, which
call the same HIP wrappers wave by wave in the reference glue's order (the
forward intermediates have the same names and meaning on both paths).
Problems with one parameter row per item (``itemwise``: G = number of items,
each clade row reading its item's rates through ``rate_item_idx``) run both
passes on the per-call drivers: the whole-pass driver covers one row.
"""

from __future__ import annotations

from types import SimpleNamespace

import torch

from kbench.api.solver_options import SolverOptions
from kbench.fused import FORWARD_SAVED_NAMES, FusedSolver

__all__ = ["FORWARD_SAVED_NAMES", "make_static", "run_forward", "run_backward", "fused_solver",
           "needs_per_call_backward", "run_forward_fused", "run_backward_fused"]


def _on_device(x, device):
    """Copy of a nested layout (dicts, lists, tuples, tensors, scalars) with every tensor on ``device``."""
    kind = type(x)
    if torch.is_tensor(x):
        return x.to(device)
    if kind is dict:
        return {k: _on_device(v, device) for k, v in x.items()}
    if kind in (list, tuple):
        return kind(_on_device(v, device) for v in x)
    return x


def make_static(captured: dict, device) -> SimpleNamespace:
    """The ``static`` namespace of a captured (or generated) problem dict, on ``device``."""
    options = SolverOptions(**dict(captured["meta"]["solver_options"]))
    options.validate()
    st = captured["static"]
    fields = {name: _on_device(st[name], device) for name in ("wave_layout", "state_helpers", "rate_item_idx")}
    return SimpleNamespace(**fields, itemwise=bool(st["itemwise"]), statewise=bool(st["statewise"]),
                           solver_options=options, warm_E=None)


def fused_solver(static) -> FusedSolver:
    """The native whole-pass solver of ``static``: created on first use and kept as an
    attribute of the static object, so it lives exactly as long as that object."""
    solver = getattr(static, "_fused_solver", None)
    if solver is None:
        solver = FusedSolver(static, static.solver_options)
        static._fused_solver = solver
    return solver


def run_forward(static, theta: torch.Tensor, col_weights: torch.Tensor):
    """theta -> (loss, saved forward intermediates)."""
    if static.itemwise:
        from kbench.percall import run_forward as run_forward_per_call

        return run_forward_per_call(static, theta, col_weights)
    with torch.no_grad():
        loss, saved = fused_solver(static).run_forward(theta, col_weights)
    saved.pop("_use_col_weights", None)
    return loss, saved


def needs_per_call_backward(static) -> bool:
    """True when the solver options ask for a backward the whole-pass driver does not implement,
    or the problem has one parameter row per item."""
    so = static.solver_options
    return (str(so.self_loop_solver).strip().lower() != "neumann"
            or float(so.pibar_side_threshold) > 0.0 or bool(static.itemwise))


def run_backward(static, theta: torch.Tensor, col_weights: torch.Tensor, saved: dict):
    """(saved forward intermediates) -> (grad_theta, grad_col); a failed E-adjoint solve raises RuntimeError."""
    if needs_per_call_backward(static):
        from kbench import percall

        return percall.run_backward(static, theta, col_weights, saved)
    with torch.no_grad():
        return fused_solver(static).run_backward(theta, col_weights, saved)


def run_backward_fused(static, theta: torch.Tensor, col_weights: torch.Tensor, saved: dict):
    """``run_backward`` on the whole-pass driver only: options it does not implement raise
    ``NotImplementedError`` instead of selecting the per-call path."""
    with torch.no_grad():
        return fused_solver(static).run_backward(theta, col_weights, saved)


def run_forward_fused(static, theta: torch.Tensor, col_weights: torch.Tensor):
    """``run_forward`` on the whole-pass driver only (``itemwise`` problems raise
    ``NotImplementedError`` instead of selecting the per-call path)."""
    with torch.no_grad():
        loss, saved = fused_solver(static).run_forward(theta, col_weights)
    saved.pop("_use_col_weights", None)
    return loss, saved
