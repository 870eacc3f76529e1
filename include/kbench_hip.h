/*
 * libkbench_hip -- C ABI of the MI355X (gfx950) log-space solver path.
 *
 * The reference (SisyphusMountain/kernel-bench) has no native FFI: its hot
 * path is Triton kernels launched from Python wrappers in
 * kbench/core/kernels/*.py.  Each entry point below replaces a group of those
 * launches; the comment on each names the reference interface (file:line,
 * paths relative to the reference root, "pristine" =
 * experiments/pristine_kernels/).
 *
 * Conventions: plain pointers and sizes only.  Pointers named in *_io structs
 * are device pointers (HIP global memory) unless noted; `stream` is a
 * hipStream_t passed as void*.  Every function returns 0 on success or a
 * negative KB_ERR_* code; kb_last_error() describes the failure of the last
 * call on the calling thread.  Nothing here synchronises the stream unless
 * its comment says so.
 */
#ifndef KBENCH_HIP_H
#define KBENCH_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KB_ABI_VERSION 4

#define KB_ERR_ARG (-1)    /* invalid argument / layout (reference raises ValueError) */
#define KB_ERR_HIP (-2)    /* HIP runtime error (reference: RuntimeError) */
#define KB_ERR_SOLVE (-3)  /* iterative solve failed (reference: RuntimeError, _implicit_grad.py:94) */

/* Message of the last failing call on this thread. */
const char* kb_last_error(void);
int kb_abi_version(void);

/*
 * Static problem layout, host pointers (read once by kb_plan_create).
 * Field meanings follow the reference's `static` namespace
 * (kbench/runtime.py:47-60): state_helpers (node_parent, node_child1/2 with a
 * >= S "no child" sentinel, node_subtree_start/end, unnorm_row_max) and
 * wave_layout (leaf_state_index, root_row_ids, wave_metas[start, W, sl, sr,
 * reduce_idx, log_split_probs]) plus rate_item_idx.  Splits are given with
 * their global parent row (wave start + reduce_idx).
 */
typedef struct kb_layout {
  int32_t S, C, n_fam, n_waves;
  const int64_t* node_parent;        /* [S], -1 at the root */
  const int64_t* node_child1;        /* [S], >= S: none */
  const int64_t* node_child2;        /* [S] */
  const int64_t* node_subtree_start; /* [S] preorder index */
  const int64_t* node_subtree_end;   /* [S] preorder index + subtree size */
  const float* unnorm_row_max;       /* [S] */
  const int64_t* leaf_state_index;   /* [C], -1 for non-leaf rows */
  const int64_t* rate_item_idx;      /* [C] */
  const int64_t* root_row_ids;       /* [n_fam] */
  const int64_t* wave_start;         /* [n_waves] */
  const int64_t* wave_size;          /* [n_waves] */
  const int32_t* wave_has_splits;    /* [n_waves] */
  int64_t n_splits;
  const int64_t* split_parent;       /* [n_splits] global parent row */
  const int64_t* split_left;         /* [n_splits] global child rows */
  const int64_t* split_right;
  const double* split_log_prob;      /* [n_splits] log2 split probability */
} kb_layout;

typedef struct kb_plan kb_plan;

/* Build the device-resident layout tables (allocates device memory). */
int kb_plan_create(const kb_layout* layout, kb_plan** out);
void kb_plan_destroy(kb_plan* plan);
/* out[0..n), n <= 13: S, C, n_fam, n_waves, pointer-jump rounds, bottom-up
 * levels, dependency levels, rows the forward computes (one per class of
 * identical rows), classes of level-0 rows, level-0 rows, kb_solve's overlap
 * cut (-1: none), the rows it solves early and the lowest level of those. */
int kb_plan_info(const kb_plan* plan, int32_t* out, int n);

/*
 * Whole forward pass: theta -> loss and the forward intermediates.
 * Replaces reference kbench/runtime.py:63-75 run_forward, i.e.
 * solver.py:16-96 solve_e_pi (extract_parameters_* + e_fixed_point_triton,
 * pristine e_step.py:438-501) -> forward.py:8-117 pi_wave_forward
 * (compute_dts_forward dts_fused.py:171-231, compute_leaf_initial_wave_step
 * wave_step.py:313-361, compute_wave_step wave_step.py:363-410) ->
 * solver.py:141-142 nll_from_root_rows.
 * One fused kernel per wave runs the split reduction and all pi_iters-1
 * sweeps with the row on chip.  Output pointers are device buffers of the
 * reference's saved-tensor shapes (runtime.py:29-32).
 */
typedef struct kb_forward_io {
  const float* theta;        /* [S,3] if statewise else [3] */
  int32_t statewise;
  const float* col_weights;  /* [S] */
  int32_t use_col_weights;   /* 0 when all col_weights are equal (solver.py:11-13) */
  double e_init;
  int32_t e_max_iter;
  double e_tol;
  int32_t pi_iters;
  float* E;                  /* [S] (item rows = 1) */
  float* E_s1;
  float* E_s2;
  float* Ebar;
  float* log_pS;             /* [S] statewise, [1] global */
  float* log_pD;
  float* log_pL;
  float* max_coupling;       /* [S] */
  float* col_log_probs;      /* [S] */
  float* pi;                 /* [C,S] pi_wave */
  float* pibar;              /* [C,S] pibar_wave */
  float* pibar_row_max;      /* [C] */
  float* loss;               /* [1] */
} kb_forward_io;

int kb_forward(kb_plan* plan, const kb_forward_io* io, void* stream);

/* Synchronises `stream`; returns the E-step iteration count and the float64 loss. */
int kb_forward_stats(kb_plan* plan, int32_t* n_e_iter, double* loss64, void* stream);

/*
 * Whole backward pass: forward intermediates -> (grad_theta, grad_col).
 * Replaces reference kbench/runtime.py:77-115 run_backward, i.e.
 * _implicit_grad.py:97-370 (per wave in reverse:
 * active_mask_from_rhs_absmax_fused wave_backward.py:168-201,
 * compute_dts_forward with active parents, wave_backward_uniform_fused
 * wave_backward.py:1398-1522, the _scatter_accum bucket sums,
 * dts_cross_backward_accum_fused wave_backward.py:1980-2190,
 * uniform_cross_pibar_vjp_tree_from_ud_fused wave_backward.py:2330-2446)
 * and _e_adjoint_and_theta_vjp _implicit_grad.py:373-475 (BiCGSTAB + VJP).
 * One fused kernel per wave; child adjoints are gathered from per-split
 * staging rows in a fixed order (no atomics), so the result is bitwise
 * reproducible.  A BiCGSTAB failure is reported by kb_backward_stats.
 */
typedef struct kb_backward_io {
  const float* theta;
  int32_t statewise;
  const float* col_weights;
  int32_t use_col_weights;
  int32_t neumann_terms;
  double pruning_threshold;
  int32_t use_pruning;
  int32_t bicgstab_max_iter;
  double bicgstab_tol;
  double bicgstab_breakdown_tol;
  const float* E;            /* saved forward tensors (kb_forward_io shapes) */
  const float* E_s1;
  const float* E_s2;
  const float* Ebar;
  const float* log_pS;
  const float* log_pD;
  const float* log_pL;
  const float* max_coupling;
  const float* col_log_probs;
  const float* pi;
  const float* pibar;
  const float* pibar_row_max;
  float* grad_theta;         /* theta's shape */
  float* grad_col;           /* [S] */
  uint8_t* active_mask;      /* optional [C] out: 1 = row active */
  double* acc_out;           /* optional [8,S] out: gradient accumulators
                                (pD, pS, E, Ebar, E_s1, E_s2, max_coupling, col) */
  int64_t forward_token;     /* kb_forward_token() of the forward that produced pi /
                                pibar, or 0: with a token that is still current the
                                split terms stored by that forward are reused instead
                                of recomputed from pi / pibar */
  double neumann_rtol;       /* 0: every row sums all neumann_terms terms (the
                                reference's series).  > 0: a row's series stops at
                                the first term n >= 1 whose every entry is at most
                                neumann_rtol * max|adjoint of the row|; that term is
                                included.  Not in the reference. */
  uint8_t* neumann_terms_out; /* optional [C] out: J^T applications of every solved
                                row (level-0 classes: at their first member);
                                untouched for other rows */
} kb_backward_io;

int kb_backward(kb_plan* plan, const kb_backward_io* io, void* stream);

/*
 * One forward and its backward in one call: what kb_forward followed by
 * kb_backward computes (reference kbench/runtime.py:63-75 run_forward, then
 * :77-115 run_backward on its outputs), with the two passes overlapped.  The
 * rows of every family whose root lies at a dependency level <= the plan's
 * overlap cut, at levels from the cut down to the window's lowest level, are
 * solved on a second stream, once the forward has passed the cut, while the
 * forward's later levels run; the other rows down to that level, then the
 * levels below it whole, level 0 and the epilogue follow on the caller's
 * stream, which has joined the second stream before kb_solve returns (in
 * stream order).  Both are chosen when the plan is created: the cut is the
 * highest level whose forward rows would not fit beside the early launches,
 * the lowest level the lowest one at which the early launches still take no
 * longer than the other stream's work beside them; -1 (two passes in order)
 * when the early launches would hold fewer rows than CUs.  Environment
 * KB_OVERLAP_CUT / KB_OVERLAP_LOW / KB_OVERLAP_GRID override the cut, the
 * lowest level and the early launches' workgroups (default 5/8 of the CUs).
 * bio must name the forward's outputs as its inputs (fio->pi etc.); its
 * forward_token is ignored.  Same outputs as the two calls, up to the order of
 * the gradient bucket sums (bitwise reproducible run to run).
 */
int kb_solve(kb_plan* plan, const kb_forward_io* fio, const kb_backward_io* bio, void* stream);

/*
 * The E adjoint of the backward's epilogue for given cotangents, without the
 * theta / column VJP: solves (I - J_E^T) w = q by BiCGSTAB (one workgroup,
 * float64, the stopping and breakdown rules of kb_backward's epilogue) with
 * q = acc_E + (E_s1, E_s2, Ebar cotangents pulled back to E) + q_extra
 * (+ the loss normaliser's E gradient when with_norm), then writes w and the
 * per-state cotangents of (log_pS, log_pD, log_pL, max_coupling,
 * col_log_probs) of one E step at (w, acc_Ebar), plus acc's pS, pD, mt and
 * col rows.  Replaces the Python BiCGSTAB of the reference's
 * _implicit_grad.py:28-94 and its E-step VJP / parameter pull-back
 * (_implicit_grad.py:373-430) where a caller solves the E adjoint for other
 * cotangents than the backward's own (the exact HVP's tangent E adjoint,
 * newton/hvp_exact.py:330-381).  One item row (itemwise=False) only.
 */
#define KB_E_ADJOINT_WORK_VECTORS 16
typedef struct kb_e_adjoint_io {
  int32_t statewise;
  int32_t use_col_weights;
  int32_t with_norm;         /* add d/dE n_fam log2(1 - mean 2^E) to q */
  int32_t bicgstab_max_iter;
  double bicgstab_tol;
  double bicgstab_breakdown_tol;
  const float* E;            /* [S] the E fixed point and the rates (kb_forward_io shapes) */
  const float* log_pS;
  const float* log_pD;
  const float* log_pL;
  const float* max_coupling;
  const float* col_log_probs;
  const double* acc;         /* [8,S] cotangents (pD, pS, E, Ebar, E_s1, E_s2, max_coupling, col) */
  const double* q_extra;     /* [S] added to q, or null */
  double* w_out;             /* [S] the E adjoint, or null */
  double* g_out;             /* [5,S] cotangents of (pS, pD, pL, max_coupling, col) per state */
  double* work;              /* [KB_E_ADJOINT_WORK_VECTORS, S] scratch */
  int32_t* status;           /* [2] device: iterations, failure flag */
} kb_e_adjoint_io;

int kb_e_adjoint(kb_plan* plan, const kb_e_adjoint_io* io, void* stream);

/* Token of the last kb_forward on this plan (a counter; 0 before the first). */
int64_t kb_forward_token(const kb_plan* plan);

/* Synchronises `stream`; BiCGSTAB iteration count; KB_ERR_SOLVE if it failed. */
int kb_backward_stats(kb_plan* plan, int32_t* n_iter, void* stream);

/*
 * Measurement hooks (no reference counterpart: the reference is timed with
 * CUDA events around whole passes, bench/_common.py:49-77).  When enabled,
 * kb_forward / kb_backward record a HIP event pair around every wave-kernel
 * launch on the launch stream; kb_profile_read returns the per-wave launch
 * durations (ms) of the last pass (which = 0 forward, 1 backward).
 */
int kb_profile_enable(kb_plan* plan, int enable);
int kb_profile_read(kb_plan* plan, int which, float* ms, int n);

#ifdef __cplusplus
}
#endif

#endif /* KBENCH_HIP_H */
