"""Entry points of the path: ``make_static``, ``run_forward``, ``run_backward``.

Same contract as the reference driver (reference kbench/runtime.py:29-115):

* ``make_static(captured, device)`` rebuilds the ``static`` namespace from a
  captured / generated dict (``meta``, ``static``);
* ``run_forward(static, theta, col_weights) -> (loss, saved)`` with the saved
  tensors named as in ``FORWARD_SAVED_NAMES``;
* ``run_backward(static, theta, col_weights, saved) -> (grad_theta, grad_col)``.

Both run the frozen-glue counterparts (``kbench.core.inference.solver`` and
``kbench.api._implicit_grad``), which call the HIP-backed wrappers of
``kbench.core.kernels`` exactly as the reference glue calls its Triton
wrappers.  ``run_forward_fused`` / ``run_backward_fused`` run the same passes
through the native whole-pass driver (``kbench.fused.FusedSolver``).
"""

from __future__ import annotations

from types import SimpleNamespace

import torch

from kbench.api.solver_options import SolverOptions

FORWARD_SAVED_NAMES = (
    "E", "E_s1", "E_s2", "Ebar", "root_rows", "pi_wave", "pibar_wave",
    "pibar_row_max", "log_pS", "log_pD", "log_pL", "max_coupling", "col_log_probs",
)


def move_to_device(obj, device):
    """Recursively move every tensor inside a nested dict/list to ``device``."""
    if torch.is_tensor(obj):
        return obj.to(device)
    if isinstance(obj, dict):
        return {k: move_to_device(v, device) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return type(obj)(move_to_device(v, device) for v in obj)
    return obj


def make_static(captured: dict, device) -> SimpleNamespace:
    """Rebuild the ``static`` object the solve and the implicit gradient expect."""
    st = captured["static"]
    solver_options = SolverOptions(**captured["meta"]["solver_options"])
    solver_options.validate()
    return SimpleNamespace(
        wave_layout=move_to_device(st["wave_layout"], device),
        state_helpers=move_to_device(st["state_helpers"], device),
        rate_item_idx=move_to_device(st["rate_item_idx"], device),
        itemwise=bool(st["itemwise"]),
        statewise=bool(st["statewise"]),
        solver_options=solver_options,
        warm_E=None,
    )


def run_forward(static, theta: torch.Tensor, col_weights: torch.Tensor):
    """theta -> (loss, dict of forward intermediates), through the glue and the wrappers."""
    from kbench.core.inference.solver import nll_from_root_rows, solve_e_pi

    with torch.no_grad():
        out = solve_e_pi(static, theta, col_weights, warm_start_E=None)
        loss = nll_from_root_rows(out[4], out[0])
    return loss, dict(zip(FORWARD_SAVED_NAMES, out))


def run_backward(static, theta, col_weights, saved: dict):
    """(forward intermediates) -> (grad_theta, grad_col), through the glue and the wrappers."""
    from kbench.api._implicit_grad import implicit_grad_loglik_vjp_wave
    from kbench.core.inference.solver import col_weights_are_uniform

    so = static.solver_options
    return implicit_grad_loglik_vjp_wave(
        static.wave_layout,
        static.state_helpers,
        Pi_star_wave=saved["pi_wave"],
        Pibar_star_wave=saved["pibar_wave"],
        E_star=saved["E"],
        Ebar=saved["Ebar"],
        E_s1=saved["E_s1"],
        E_s2=saved["E_s2"],
        log_pS=saved["log_pS"],
        log_pD=saved["log_pD"],
        log_pL=saved["log_pL"],
        max_coupling_mat=saved["max_coupling"],
        col_log_probs=saved["col_log_probs"],
        use_col_weights=not col_weights_are_uniform(col_weights),
        theta=theta,
        col_weights=col_weights,
        item_idx=static.rate_item_idx,
        uniform_pibar_row_max=saved["pibar_row_max"],
        statewise=static.statewise,
        itemwise=static.itemwise,
        neumann_terms=so.neumann_terms,
        self_loop_solver=so.self_loop_solver,
        bicgstab_max_iter=so.bicgstab_max_iter,
        bicgstab_tol=so.bicgstab_tol,
        bicgstab_breakdown_tol=so.bicgstab_breakdown_tol,
        adjoint_pruning_threshold=so.adjoint_pruning_threshold,
        use_adjoint_pruning=so.use_adjoint_pruning,
        pibar_side_threshold=so.pibar_side_threshold,
    )


_FUSED_CACHE: dict = {}


def fused_solver(static):
    """The (cached) native whole-pass solver of ``static``."""
    from kbench.fused import FusedSolver

    key = id(static)
    hit = _FUSED_CACHE.get(key)
    if hit is None or hit[0] is not static:
        solver = FusedSolver(static, static.solver_options)
        _FUSED_CACHE[key] = (static, solver)
        return solver
    return hit[1]


def run_forward_fused(static, theta, col_weights):
    """``run_forward`` through the native whole-pass driver."""
    with torch.no_grad():
        loss, saved = fused_solver(static).run_forward(theta, col_weights)
    saved.pop("_use_col_weights", None)
    return loss, saved


def run_backward_fused(static, theta, col_weights, saved):
    """``run_backward`` through the native whole-pass driver."""
    with torch.no_grad():
        return fused_solver(static).run_backward(theta, col_weights, saved)
