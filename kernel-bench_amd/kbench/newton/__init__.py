"""Second-order drivers above the solve: Krylov solvers and Newton-type optimisers.

``krylov``: CG, CG with a negative-curvature certificate, Steihaug trust-region
CG, Lanczos extremal eigenvalues (reference newton/cg.py).  ``drivers``: damped
Newton-CG, trust-region Newton and Lanczos / witness Newton over an
``Objective`` (reference newton/newton_cg.py).  ``hvp``: the exact and
Gauss-Newton Hessian-vector products over the per-call wrappers
(``make_exact_hvp``, reference newton/hvp_exact.py; ``make_ggn_hvp``,
reference newton/ggn.py).
"""

from .drivers import Objective, newton_cg, newton_lanczos, newton_tr  # noqa: F401
from .hvp import HvpPlan, TangentForward, make_exact_hvp, make_ggn_hvp  # noqa: F401
from .krylov import cg_solve, cg_witness, lanczos_extremes, lanczos_min_eigpair, steihaug_cg  # noqa: F401
