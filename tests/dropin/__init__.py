"""Drivers that call the drop-in wrappers in the reference glue's call sequence.

The reference's frozen glue (its kbench/runtime.py -> kbench/core/inference ->
kbench/api/_implicit_grad.py, and newton/{forward_tangent,hvp_exact}.py for the
exact HVP) is not part of this repository.  These drivers exist to exercise
the HIP-backed wrappers of ``kbench.core.kernels`` the way that glue does:
same wrapper functions, same arguments, same order per wave (the calls are
listed in each driver's docstring with the reference lines they mirror).

* ``solve``: ``SolvePlan`` -- forward (E fixed point, per-wave split term and
  ``pi_iters - 1`` sweeps, loss) and backward (per-wave adjoint in reverse,
  E adjoint, theta / column VJP);
* ``hvp``: ``HvpPlan`` -- the exact Hessian-vector product (forward tangent,
  tangent adjoint sweep, E side, parameter head);
* ``kernels``: the wrapper namespaces a plan calls through (the real wrappers,
  no-op stand-ins for the glue-floor measurement, a recorder for
  capture / replay).
"""

from .solve import SolvePlan, run_backward, run_forward  # noqa: F401
