"""Per-call drivers: the solve driven one wrapper call at a time, in the reference glue's call sequence.

The reference's frozen glue (its kbench/runtime.py -> kbench/core/inference ->
kbench/api/_implicit_grad.py) is not part of this package.  These drivers call
the HIP-backed wrappers of ``kbench.core.kernels`` the way that glue does:
same wrapper functions, same arguments, same order per wave (the calls are
listed in each driver's docstring with the reference lines they mirror).
``kbench.runtime`` runs its backward here for the options the whole-pass
driver does not implement (GMRES self-loop solves, a positive
``pibar_side_threshold``), and the Hessian-vector products of
``kbench.newton.hvp`` run over the same plan.

* ``solve``: ``SolvePlan`` -- forward (E fixed point, per-wave split term and
  ``pi_iters - 1`` sweeps, loss) and backward (per-wave adjoint in reverse,
  E adjoint, theta / column VJP);
* ``graph``: ``GraphedSolve`` -- the same forward and reverse wave loops
  captured once as two HIP graphs and replayed (the E adjoint stays eager);
* ``krylov``: the E adjoint's BiCGSTAB (the reference's stopping and
  breakdown rules);
* ``kernels``: the wrapper namespaces a plan calls through (the real wrappers,
  and no-op stand-ins that time the driver alone).
"""

from .graph import GraphedSolve  # noqa: F401
from .solve import SolvePlan, plan_of, run_backward, run_forward  # noqa: F401
