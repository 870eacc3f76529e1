"""Second-order (Newton) glue over the HIP-backed kernels.

Counterpart of the reference's top-level ``newton`` package for the pieces on
the solver's hot path: ``forward_tangent.jvp_root_scores`` (the forward-mode
tangent of the root rows, reference newton/forward_tangent.py).
"""
