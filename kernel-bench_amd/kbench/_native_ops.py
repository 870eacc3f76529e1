"""ctypes declarations of the per-wrapper entry points (include/kbench_ops.h).

Field order and types mirror the C structs exactly; every pointer is a device
address (``int``) unless the header says otherwise.
"""

from __future__ import annotations

import ctypes as ct

i32 = ct.c_int32
i64 = ct.c_int64
f64 = ct.c_double
vp = ct.c_void_p
P_i64 = ct.POINTER(ct.c_int64)

KB_F32, KB_F64, KB_BF16 = 0, 1, 2


def _ptrs(*names):
    return [(n, vp) for n in names]


class KbEStepIO(ct.Structure):
    _fields_ = [("dtype", i32), ("G", i32), ("mode", i32), ("use_col_weights", i32), ("max_iter", i32),
                ("tol", f64)] + _ptrs("E", "log_pS", "log_pD", "log_pL", "max_coupling", "col_log_probs",
                                      "E_out", "E_s1", "E_s2", "Ebar", "max_diff", "n_iter")


class KbEStepVjpIO(ct.Structure):
    _fields_ = [("dtype", i32), ("G", i32), ("use_col_weights", i32)] + _ptrs(
        "E", "E_new", "E_s1", "E_s2", "Ebar", "log_pS", "log_pD", "log_pL", "col_log_probs",
        "g_E_new", "g_E_s1", "g_E_s2", "g_Ebar",
        "grad_E", "grad_log_pS", "grad_log_pD", "grad_log_pL", "grad_max_coupling", "grad_col_log_probs", "work")


class KbWaveStepIO(ct.Structure):
    _fields_ = [("dtype", i32), ("S", i32), ("W", i32), ("use_col_weights", i32), ("use_leaf_index", i32),
                ("store_final_pibar", i32), ("n_sweeps", i32), ("ws", i64), ("pi_ws", i64),
                ("const_stride", i64)] + _ptrs(
        "Pi_in", "Pi_out", "Pibar", "pibar_row_max", "pi_residual", "dts",
        "max_coupling", "DL", "Ebar", "E", "SL1", "SL2", "col_log_probs", "item_idx", "leaf_state", "leaf_logp")


class KbLeafInitIO(ct.Structure):
    _fields_ = [("dtype", i32), ("S", i32), ("W", i32), ("use_col_weights", i32), ("ws", i64),
                ("const_stride", i64)] + _ptrs(
        "node_child1", "node_child2", "Pi_out", "max_coupling", "DL", "Ebar", "E", "SL1", "SL2", "col_log_probs",
        "subtree_start", "subtree_end", "item_idx", "leaf_state", "leaf_logp")


class KbDtsIO(ct.Structure):
    _fields_ = [("dtype", i32), ("S", i32), ("W", i32), ("param_by_state", i32), ("N", i64),
                ("item_offset", i64), ("param_row_stride", i64)] + _ptrs(
        "node_child1", "node_child2", "Pi", "Pibar", "sl", "sr", "log_split_probs", "split_ptr", "split_order",
        "log_pD", "log_pS", "item_idx", "active", "out")


class KbWaveBwdIO(ct.Structure):
    _fields_ = [("dtype", i32), ("S", i32), ("W", i32), ("n_terms", i32), ("const_layout", i32),
                ("leaf_mode", i32), ("use_leaf_index", i32), ("use_col_weights", i32), ("ws", i64)] + _ptrs(
        "Pi", "Pibar", "pibar_row_max", "dts", "rhs", "initial_v", "active", "max_coupling", "DL", "Ebar", "E", "SL1", "SL2",
        "col_log_probs", "item_idx", "leaf_state", "leaf_logp", "leaf_term",
        "v", "aw0", "aw1", "aw2", "aw345", "aw3", "aw4", "col_rows", "relres")


class KbDtsCrossIO(ct.Structure):
    _fields_ = [("dtype", i32), ("S", i32), ("param_layout", i32), ("mt_layout", i32), ("output_ud", i32),
                ("skip_inactive_ud_zero", i32), ("N", i64), ("ws", i64), ("side_threshold", f64)] + _ptrs(
        "node_child1", "node_child2", "Pi", "Pibar", "v", "active", "sl", "sr", "reduce_idx", "wlsp",
        "log_pD", "log_pS", "item_idx", "mt", "pibar_row_max", "side_rows", "ud", "A", "side_active",
        "grad_Pibar_l", "grad_Pibar_r", "param_rows", "param_sums", "mt_rows")


class KbPibarVjpIO(ct.Structure):
    _fields_ = [("dtype", i32), ("S", i32), ("use_col_weights", i32), ("N", i64)] + _ptrs(
        "Pi", "col_log_probs", "ud", "A", "side_active", "sl", "sr", "reduce_idx", "active", "pibar_row_max",
        "contrib")


class KbETanIO(ct.Structure):
    _fields_ = [("dtype", i32), ("G", i32), ("use_col_weights", i32), ("max_iter", i32), ("tol", f64)] + _ptrs(
        "E", "log_pS", "log_pD", "log_pL", "max_coupling", "col_log_probs", "dlog_pS", "dlog_pD", "dlog_pL",
        "dmax_coupling", "dE0", "dE", "dE_s1", "dE_s2", "dEbar", "n_iter")


class KbDtsTanIO(ct.Structure):
    _fields_ = [("dtype", i32), ("S", i32), ("W", i32), ("param_by_state", i32), ("N", i64),
                ("item_offset", i64), ("param_row_stride", i64)] + _ptrs(
        "node_child1", "node_child2", "Pi", "Pibar", "dPi", "dPibar", "sl", "sr", "log_split_probs", "split_ptr",
        "split_order", "log_pD", "log_pS", "dlog_pD", "dlog_pS", "dts_r", "item_idx", "out")


class KbWaveTanIO(ct.Structure):
    _fields_ = [("dtype", i32), ("S", i32), ("W", i32), ("use_col_weights", i32), ("use_leaf_index", i32),
                ("n_iters", i32), ("ws", i64), ("pi_ws", i64), ("const_stride", i64)] + _ptrs(
        "Pi_in", "dPi_in", "dPi_out", "dPibar_out", "dts", "d_dts", "max_coupling", "dMC", "DL", "dDL", "Ebar",
        "dEbar", "E", "dE", "SL1", "dSL1", "SL2", "dSL2", "col_log_probs", "item_idx", "leaf_state", "leaf_logp",
        "dleaf_logp")


class KbEStepSoIO(ct.Structure):
    _fields_ = [("dtype", i32), ("G", i32), ("use_col_weights", i32)] + _ptrs(
        "E", "E_new", "E_s1", "E_s2", "Ebar", "log_pS", "log_pD", "log_pL", "col_log_probs", "g_new", "g_ebar",
        "dE", "dE_new", "dE_s1", "dE_s2", "dEbar", "dlog_pS", "dlog_pD", "dlog_pL", "dcol",
        "d_grad_E", "d_grad_pS", "d_grad_pD", "d_grad_pL", "d_grad_mc", "col_rows")


class KbWaveSoIO(ct.Structure):
    _fields_ = [("dtype", i32), ("S", i32), ("W", i32), ("use_col_weights", i32), ("use_leaf_index", i32),
                ("ws", i64), ("const_stride", i64)] + _ptrs(
        "Pi", "dPi", "Pibar", "dPibar", "v", "pibar_row_max", "DL", "dDL", "Ebar", "dEbar", "E", "dE", "SL1", "dSL1",
        "SL2", "dSL2", "col_log_probs", "item_idx", "leaf_state", "leaf_logp", "dleaf_logp", "dts", "d_dts", "d_rhs",
        "d_out", "d_aw0", "d_aw1", "d_aw2", "d_aw345", "d_aw3", "d_aw4")


class KbDtsSoIO(ct.Structure):
    _fields_ = [("dtype", i32), ("S", i32), ("param_by_state", i32), ("use_col_weights", i32), ("N", i64),
                ("ws", i64), ("item_offset", i64), ("param_row_stride", i64), ("mt_row_stride", i64)] + _ptrs(
        "Pi", "dPi", "Pibar", "dPibar", "v", "sl", "sr", "reduce_idx", "log_split_probs", "log_pD", "log_pS",
        "dlog_pD", "dlog_pS", "mt", "dmt", "item_idx", "pibar_row_max", "col_log_probs", "node_child1",
        "node_child2", "ud", "dud", "side_rows", "col_rows", "pD_rows", "pS_rows", "mt_rows")


def declare(lib) -> None:
    def fn(name, argtypes, restype=ct.c_int):
        f = getattr(lib, name)
        f.argtypes = argtypes
        f.restype = restype

    fn("kb_tree_create", [i32, P_i64, P_i64, P_i64, ct.POINTER(vp)])
    fn("kb_tree_destroy", [vp], None)
    fn("kb_ops_max_states", [ct.c_int])
    fn("kb_estep", [vp, ct.POINTER(KbEStepIO), vp])
    fn("kb_estep_vjp", [vp, ct.POINTER(KbEStepVjpIO), vp])
    fn("kb_estep_vjp_noalloc", [vp, ct.POINTER(KbEStepVjpIO), vp])
    fn("kb_wave_step", [vp, ct.POINTER(KbWaveStepIO), vp])
    fn("kb_leaf_init", [ct.POINTER(KbLeafInitIO), vp])
    fn("kb_dts_forward", [ct.POINTER(KbDtsIO), vp])
    fn("kb_active_mask", [i32, i32, i32, i64, vp, ct.c_float, i32, vp, vp])
    fn("kb_wave_backward", [vp, ct.POINTER(KbWaveBwdIO), vp])
    fn("kb_dts_cross_backward", [ct.POINTER(KbDtsCrossIO), vp])
    fn("kb_pibar_vjp", [vp, ct.POINTER(KbPibarVjpIO), vp])
    fn("kb_rows_scatter_add", [i32, i32, i64, vp, vp, vp, vp, i64, vp])
    fn("kb_rows_sum_into", [i32, i32, i64, vp, vp, vp, vp])
    fn("kb_rows_sum_multi", [i32, i32, i64, i32, ct.POINTER(vp), ct.POINTER(vp), vp, vp, vp])
    fn("kb_rows_sum_accum", [i32, i32, i32, ct.POINTER(i64), ct.POINTER(i32), ct.POINTER(vp), ct.POINTER(vp), vp,
                             vp])
    fn("kb_e_tangent_fixed_point", [vp, ct.POINTER(KbETanIO), vp])
    fn("kb_dts_tangent", [ct.POINTER(KbDtsTanIO), vp])
    fn("kb_wave_step_tangent", [vp, ct.POINTER(KbWaveTanIO), vp])
    fn("kb_estep_backward_so", [vp, ct.POINTER(KbEStepSoIO), vp])
    fn("kb_wave_backward_so", [vp, ct.POINTER(KbWaveSoIO), vp])
    fn("kb_dts_backward_so", [vp, ct.POINTER(KbDtsSoIO), vp])
