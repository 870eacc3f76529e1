"""HIP-backed drop-in replacements of the reference's kbench/core/kernels wrappers.

Modules and the reference modules they replace (same function names and
signatures):

* ``e_step`` -- e_step.py (``e_step_triton_autograd``, ``e_fixed_point_triton``)
* ``wave_step`` -- wave_step.py (``compute_leaf_initial_wave_step``, ``compute_wave_step``)
* ``dts_fused`` -- dts_fused.py (``compute_dts_forward``)
* ``wave_backward`` -- wave_backward.py (``active_mask_from_rhs_absmax_fused``,
  ``wave_backward_uniform_fused``, ``dts_cross_backward_accum_fused``,
  ``uniform_cross_pibar_vjp_tree_from_ud_fused``)
* ``e_step_tangent`` -- e_step_tangent.py (``e_tangent_fixed_point``)
* ``dts_tangent`` -- dts_tangent.py (``compute_dts_tangent``)
* ``wave_tangent`` -- wave_tangent.py (``compute_wave_step_tangent``,
  ``compute_wave_step_tangent_selfloop``)
* ``e_step_so`` -- e_step_so.py (``e_step_backward_so``)
* ``wave_so`` -- wave_so.py (``wave_backward_so``)
* ``dts_so`` -- dts_so.py (``dts_backward_so``)
* ``_dts_layout_contract`` -- _dts_layout_contract.py (host-side layout codes)

The native launchers are declared in include/kbench_ops.h.
"""
