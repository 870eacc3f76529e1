/*
 * libkbench_hip -- per-wrapper entry points.
 *
 * The reference's hot path is a set of Triton launches behind the Python
 * wrappers in kbench/core/kernels/*.py, which the frozen glue
 * (kbench/core/inference/forward.py, solver.py, kbench/api/_implicit_grad.py)
 * imports by name.  The functions below are the native launchers beneath a
 * drop-in replacement of each wrapper; each comment names the reference
 * function it replaces (paths relative to the reference root; "pristine" =
 * experiments/pristine_kernels/, identical to kbench/core/kernels/ for these
 * files).
 *
 * Conventions (shared with kbench_hip.h):
 *  - plain device pointers, sizes and flags; `stream` is a hipStream_t as void*;
 *  - `dtype` selects the element type of every floating-point tensor of the
 *    call: KB_F32 or KB_F64 (the reference's DTYPE constexpr);
 *  - [R, S] tensors are dense row-major (row stride S);
 *  - index tensors are int64 unless named *_i32;
 *  - return 0 or a negative KB_ERR_* code, kb_last_error() has the message;
 *  - nothing synchronises the stream; there are no atomics: every reduction
 *    is done in a fixed order, so results are bitwise reproducible.
 *
 * Scratch buffers (`work*` arguments) are device memory the caller provides;
 * the sizes are given per function.
 */
#ifndef KBENCH_OPS_H
#define KBENCH_OPS_H

#include <stdint.h>

#include "kbench_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define KB_F32 0
#define KB_F64 1

/*
 * Species-tree tables for the per-wrapper kernels (preorder, Euler tour, depth
 * levels), built from the reference's state_helpers arrays (host pointers):
 * node_parent [S] (-1 at the root), node_child1/2 [S] (a value outside [0, S)
 * means "no child").  Replaces the per-launch ancestor chase bounded by
 * max_ancestor_depth and the compact_level_* tables (pristine
 * wave_step.py:52-88, wave_backward.py:479-512): both describe the same tree.
 */
typedef struct kb_tree kb_tree;
int kb_tree_create(int32_t S, const int64_t* node_parent, const int64_t* node_child1, const int64_t* node_child2,
                   kb_tree** out);
void kb_tree_destroy(kb_tree* tree);
/* Largest S the row kernels accept for `dtype` (LDS capacity). */
int kb_ops_max_states(int dtype);

/*
 * One E-step or the whole E fixed point, G item rows of S states.
 * mode 0: one step (pristine e_step.py:12-99 _e_step_forward_2d_kernel via
 *         _launch_e_step_forward_2d, 244-278); max_diff [G] (nullable) gets
 *         max_s |E_new - E|.
 * mode 1: fixed point (pristine e_step.py:438-501 e_fixed_point_triton):
 *         iterate from E until max_s |E_new - E| < tol (each item row stops on
 *         its own) or max_iter steps; E_out is the last iterate and
 *         E_s1/E_s2/Ebar are evaluated at it.  n_iter [G] (nullable, int32).
 * Arithmetic is float64 whatever `dtype`.
 */
typedef struct kb_estep_io {
  int32_t dtype, G, mode, use_col_weights, max_iter;
  double tol;
  const void* E;                                   /* [G, S] */
  const void *log_pS, *log_pD, *log_pL, *max_coupling; /* [G, S] */
  const void* col_log_probs;                       /* [S] */
  void *E_out, *E_s1, *E_s2, *Ebar;                /* [G, S] */
  void* max_diff;                                  /* [G] or NULL */
  int32_t* n_iter;                                 /* [G] or NULL */
} kb_estep_io;
int kb_estep(const kb_tree* tree, const kb_estep_io* io, void* stream);

/*
 * VJP of one E-step (pristine e_step.py:102-241 prepare/finalize kernels,
 * _TritonEStep2D.backward 313-407): cotangents of (E_new, E_s1, E_s2, Ebar)
 * -> gradients wrt E, log_pS, log_pD, log_pL, max_coupling ([G, S] each)
 * and col_log_probs ([S]: the sum over item rows, in row order, is added
 * into grad_col_log_probs, which the caller zeroes as the reference does).
 * work: G * S doubles.  Float64 arithmetic.
 */
typedef struct kb_estep_vjp_io {
  int32_t dtype, G, use_col_weights;
  const void *E, *E_new, *E_s1, *E_s2, *Ebar;      /* [G, S] forward values */
  const void *log_pS, *log_pD, *log_pL;            /* [G, S] */
  const void* col_log_probs;                       /* [S] */
  const void *g_E_new, *g_E_s1, *g_E_s2, *g_Ebar;  /* [G, S] cotangents */
  void *grad_E, *grad_log_pS, *grad_log_pD, *grad_log_pL, *grad_max_coupling; /* [G, S] */
  void* grad_col_log_probs;                        /* [S] */
  double* work;                                    /* [G, S] */
} kb_estep_vjp_io;
int kb_estep_vjp(const kb_tree* tree, const kb_estep_vjp_io* io, void* stream);

/*
 * kb_estep_vjp without a work buffer and without any device allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight solver loops such as the
 * E-adjoint BiCGSTAB, harnesses that forbid hipMalloc).  io->work must be NULL;
 * the [G, S] float64 staging rows live in a device array of the library,
 * KB_ESTEP_VJP_NOALLOC_MAX doubles (512 KiB) on each GPU for the life of the
 * process, so G * S must not exceed KB_ESTEP_VJP_NOALLOC_MAX (else KB_ERR_ARG).
 * Same kernels and results as kb_estep_vjp.  Every call on one GPU shares that
 * array: calls that overlap on one GPU (concurrent streams, or host threads)
 * race and must be serialised by the caller.
 */
#define KB_ESTEP_VJP_NOALLOC_MAX 65536
int kb_estep_vjp_noalloc(const kb_tree* tree, const kb_estep_vjp_io* io, void* stream);

/*
 * Self-loop constants addressing, shared by the wave kernels: constant row
 * of wave row w is  const + item_idx[ws + w] * const_stride  (const_stride 0:
 * one shared row), as the reference's CONST_ROW_STRIDE (pristine
 * wave_step.py:10-13).
 */

/*
 * compute_wave_step (pristine wave_step.py:363-410, kernel 92-220): one
 * self-loop sweep over rows [ws, ws + W).  Input row w is Pi_in row
 * pi_ws + w (pi_ws = input_ws, or ws); output row Pi_out row ws + w.  With
 * dts (nullable) the split term of row w joins the LSE.  store_final_pibar
 * also writes Pibar row ws + w and pibar_row_max[ws + w] from the new row;
 * pi_residual (nullable, float32 [C]) gets max |Pi_new - Pi_in| over finite
 * entries.  In-place use (Pi_in == Pi_out, Pi_out == Pibar) is allowed.
 * n_sweeps > 1 runs that many sweeps in one launch with the row kept on chip
 * (bitwise equal to n_sweeps one-sweep calls chained through Pi_out; only the
 * last sweep is written, and pi_residual is the last sweep's); 0 or 1 is one.
 */
typedef struct kb_wave_step_io {
  int32_t dtype, S, W, use_col_weights, use_leaf_index, store_final_pibar, n_sweeps;
  int64_t ws, pi_ws, const_stride;
  const void* Pi_in;                               /* [*, S] */
  void* Pi_out;                                    /* [C, S] (rows ws..ws+W written) */
  void* Pibar;                                     /* [C, S] */
  void* pibar_row_max;                             /* [C] */
  float* pi_residual;                              /* [C] or NULL */
  const void* dts;                                 /* [W, S] or NULL */
  const void *max_coupling, *DL, *Ebar, *E, *SL1, *SL2; /* constant rows */
  const void* col_log_probs;                       /* [S] */
  const int64_t* item_idx;                         /* [C] */
  const int64_t* leaf_state;                       /* [C] */
  const void* leaf_logp;                           /* [G, S] (row item_idx * S) */
} kb_wave_step_io;
int kb_wave_step(const kb_tree* tree, const kb_wave_step_io* io, void* stream);

/*
 * compute_leaf_initial_wave_step (pristine wave_step.py:313-361, kernel
 * 223-310): leaf initialisation of rows [ws, ws + W) into Pi_out rows.
 */
typedef struct kb_leaf_init_io {
  int32_t dtype, S, W, use_col_weights;
  int64_t ws, const_stride;
  const int64_t *node_child1, *node_child2;        /* [S] */
  void* Pi_out;                                    /* [C, S] */
  const void *max_coupling, *DL, *Ebar, *E, *SL1, *SL2;
  const void* col_log_probs;                       /* [S] */
  const int64_t *subtree_start, *subtree_end;      /* [S] */
  const int64_t* item_idx;                         /* [C] */
  const int64_t* leaf_state;                       /* [C] */
  const void* leaf_logp;                           /* [G, S] */
} kb_leaf_init_io;
int kb_leaf_init(const kb_leaf_init_io* io, void* stream);

/*
 * compute_dts_forward (pristine dts_fused.py:171-231): out[w] = LSE over the
 * splits of row w of the five DTL split terms; -inf for rows without splits
 * and, with `active` (nullable, bool [W]), for inactive rows.  Splits are
 * grouped by row with split_ptr [W+1] / split_order [N] (int32, increasing
 * split index within a row), which gives the eq1/ge2 result of the reference
 * in one pass.  log_pD/log_pS: row item_idx[item_offset + w] * param_row_stride,
 * indexed by state when param_by_state.
 */
typedef struct kb_dts_io {
  int32_t dtype, S, W, param_by_state;
  int64_t N, item_offset, param_row_stride;
  const int64_t *node_child1, *node_child2;        /* [S] */
  const void *Pi, *Pibar;                          /* [C, S] */
  const int64_t *sl, *sr;                          /* [N] global child rows */
  const void* log_split_probs;                     /* [N] */
  const int32_t *split_ptr, *split_order;          /* [W + 1], [N] */
  const void *log_pD, *log_pS;
  const int64_t* item_idx;                         /* [C] */
  const uint8_t* active;                           /* [W] or NULL */
  void* out;                                       /* [W, S] */
} kb_dts_io;
int kb_dts_forward(const kb_dts_io* io, void* stream);

/*
 * active_mask_from_rhs_absmax_fused (pristine wave_backward.py:138-201):
 * active[w] = max_s |rhs[w, s]| >= threshold (> when strict).  dtype may also
 * be KB_BF16.
 */
#define KB_BF16 2
int kb_active_mask(int32_t dtype, int32_t W, int32_t S, int64_t row_stride, const void* rhs, float threshold,
                   int32_t strict, uint8_t* active, void* stream);

/*
 * wave_backward_uniform_fused, Neumann solver (pristine
 * wave_backward.py:1398-1522 -> 969-1395): self-loop adjoint v (rhs plus
 * n_terms applications of J^T at Pi*) of rows [ws, ws + W), and the
 * per-element parameter contributions aw0, aw1, aw2, aw345, aw3, aw4.
 * With initial_v (nullable) the solve is instead n_terms steps of
 * v <- rhs + J^T v from v = initial_v (the reference's initial_v path).
 * Inactive rows (active[w] == 0) are zero in every output.  col_rows [W, S]
 * receives each row's contribution to grad_col_log_probs (the caller sums
 * the rows), relres (nullable, float [W]) the last-increment ratio
 * ||term_n|| / ||v|| (return_last_increment).
 * const_layout: 0 shared [S], 1 row-expanded [W, S], 2 [G, S] via item_idx.
 * leaf_mode: 0 [S] shared, 1 [G] item scalar, 2 [G, S], 3 scalar; only with
 * use_leaf_index; otherwise leaf_term (nullable, [W, S]) is the materialised
 * leaf term.
 */
typedef struct kb_wave_bwd_io {
  int32_t dtype, S, W, n_terms, const_layout, leaf_mode, use_leaf_index, use_col_weights;
  int64_t ws;
  const void *Pi, *Pibar;                          /* [C, S] */
  const void* pibar_row_max;                       /* [C] */
  const void* dts;                                 /* [W, S] or NULL */
  const void* rhs;                                 /* [W, S] */
  const void* initial_v;                           /* [W, S] or NULL */
  const uint8_t* active;                           /* [W] or NULL */
  const void *max_coupling, *DL, *Ebar, *E, *SL1, *SL2;
  const void* col_log_probs;                       /* [S] */
  const int64_t* item_idx;                         /* [C] */
  const int64_t* leaf_state;                       /* [C] */
  const void* leaf_logp;
  const void* leaf_term;                           /* [W, S] or NULL */
  void *v, *aw0, *aw1, *aw2, *aw345, *aw3, *aw4;   /* [W, S] */
  void* col_rows;                                  /* [W, S] */
  float* relres;                                   /* [W] or NULL */
} kb_wave_bwd_io;
int kb_wave_backward(const kb_tree* tree, const kb_wave_bwd_io* io, void* stream);

/*
 * dts_cross_backward_accum_fused (pristine wave_backward.py:1980-2190, kernel
 * 1529-1945): per split n of the wave, the five split-term weights
 * w_k = 2^(lsp + d_k - Pi*[parent]) and vd_k = v[parent] w_k.  Writes
 *   side_rows [2N, S]: rows n / N + n are the split's contribution to the
 *     adjoint rows of its left / right child (vd0 + vd1 / vd0 + vd2 plus the
 *     speciation terms at the child columns); the caller adds them into
 *     accumulated_rhs;
 *   with output_ud: ud [2N, S] (vd2 / vd1 scaled by 2^(rowmax + mt - Pibar)),
 *     A [2N] (row sums), side_active [2N] (nullable; abs-sum > side_threshold,
 *     or any nonzero when side_threshold <= 0);
 *   without: grad_Pibar_l / grad_Pibar_r [N, S] = vd2 / vd1;
 *   param_rows [2N, S] (nullable): vd0 / vd3 + vd4 per split;
 *   param_sums [2N] (nullable): their row sums;
 *   mt_rows [2N, S] (nullable): vd2 / vd1 (left / right child side).
 * Splits of inactive parents write zeros (ud / A untouched when
 * skip_inactive_ud_zero, as the reference's SKIP_INACTIVE_PIBAR_OUTPUT_ZERO).
 * param_layout: 0 scalar [1], 1 [S], 2 [G] by parent item, 3 [G, S].
 * mt_layout: 0 [S], 1 [G, S] by child item.
 */
typedef struct kb_dts_cross_io {
  int32_t dtype, S, param_layout, mt_layout, output_ud, skip_inactive_ud_zero;
  int64_t N, ws;
  double side_threshold;
  const int64_t *node_child1, *node_child2;        /* [S] */
  const void *Pi, *Pibar;                          /* [C, S] */
  const void* v;                                   /* [W, S] */
  const uint8_t* active;                           /* [W] or NULL */
  const int64_t *sl, *sr, *reduce_idx;             /* [N] */
  const void* wlsp;                                /* [N] */
  const void *log_pD, *log_pS;
  const int64_t* item_idx;                         /* [C] or NULL */
  const void* mt;                                  /* mt_layout rows, or NULL */
  const void* pibar_row_max;                       /* [C] or NULL */
  void* side_rows;                                 /* [2N, S] */
  void *ud, *A;                                    /* [2N, S], [2N] */
  uint8_t* side_active;                            /* [2N] or NULL */
  void *grad_Pibar_l, *grad_Pibar_r;               /* [N, S] */
  void* param_rows;                                /* [2N, S] or NULL */
  void* param_sums;                                /* [2N] or NULL */
  void* mt_rows;                                   /* [2N, S] or NULL */
} kb_dts_cross_io;
int kb_dts_cross_backward(const kb_dts_cross_io* io, void* stream);

/*
 * uniform_cross_pibar_vjp_tree_from_ud_fused (pristine
 * wave_backward.py:2330-2446, kernel 2229-2327): for each split side r of
 * 2N (left sides first), skipped when side_active[r] == 0 or the parent row
 * is inactive: ud row r is replaced in place by its subtree sums and
 * contrib row r = p'(child) * (A[r] - subtree(ud)), p' = 2^((col +) Pi*[child]
 * - rowmax[child]).  Skipped sides get a zero contrib row; the caller adds
 * contrib rows into accumulated_rhs[child] and grad_col_log_probs.
 */
typedef struct kb_pibar_vjp_io {
  int32_t dtype, S, use_col_weights;
  int64_t N;
  const void* Pi;                                  /* [C, S] */
  const void* col_log_probs;                       /* [S] */
  void* ud;                                        /* [2N, S] in/out */
  const void* A;                                   /* [2N] */
  const uint8_t* side_active;                      /* [2N] or NULL */
  const int64_t *sl, *sr, *reduce_idx;             /* [N] */
  const uint8_t* active;                           /* [W] or NULL */
  const void* pibar_row_max;                       /* [C] */
  void* contrib;                                   /* [2N, S] */
} kb_pibar_vjp_io;
int kb_pibar_vjp(const kb_tree* tree, const kb_pibar_vjp_io* io, void* stream);

/*
 * Deterministic scatter-add of rows: for each run of equal keys in
 * keys_sorted (ascending; negative keys skipped), dst[key * dst_stride + s]
 * += sum over the run, in order, of src[order[j] * S + s].  Replaces the
 * reference's tl.atomic_add accumulations into accumulated_rhs, grad_mt,
 * grad_log_pD/pS (pristine wave_backward.py:1747-1853, 2320-2327).
 */
int kb_rows_scatter_add(int32_t dtype, int32_t S, int64_t n, const void* src, const int32_t* order,
                        const int64_t* keys_sorted, void* dst, int64_t dst_stride, void* stream);

/*
 * dst[s] += sum over r < n of src[r * S + s] (fixed order, float64 partial
 * sums; work: ceil(n / 64) * S doubles).  Replaces atomic column reductions
 * into grad_col_log_probs (pristine wave_backward.py:700-733, 2320-2327).
 */
int kb_rows_sum_into(int32_t dtype, int32_t S, int64_t n, const void* src, void* dst, double* work, void* stream);

/*
 * Column sums of m <= 8 row blocks in one launch (two above 64 rows):
 * out[j * S + s] = sum over r < n of (a[j][r * S + s] + b[j][r * S + s]),
 * b (or b[j]) null for a single addend, in row order with float64 partial
 * sums (work: m * ceil(n / 64) * S doubles, unused for n <= 64).  a and b
 * are host arrays of device pointers.  No reference kernel: it replaces the
 * glue's per-wave torch reductions of the aw tensors
 * (kbench/api/_implicit_grad.py:288-296, one .sum(0) per tensor).
 */
int kb_rows_sum_multi(int32_t dtype, int32_t S, int64_t n, int32_t m, const void* const* a, const void* const* b,
                      void* out, double* work, void* stream);

/*
 * Column sums of m <= 8 row blocks, each added into its own accumulator:
 * dst[j][s] += sum over r < n[j] of (a[4j][r*S+s] + ... + a[4j+k[j]-1][r*S+s])
 * with k[j] in 1..4 addends per block (each row's addends summed first, in
 * order), rows summed in order in float64 (work: m * max_j ceil(n[j] / 64) * S
 * doubles, unused when every block has at most 64 rows).  The accumulators
 * must be distinct.  n, k, a and dst are host arrays (a: 4 entries per block,
 * device pointers).  A block of one addend gives dst exactly what
 * kb_rows_sum_into gives.  No reference kernel: it replaces the per-wave
 * sequences of fixed-order sums (and the adds folding their results) that
 * stand in for the reference's atomic accumulations into grad_log_pD / pS /
 * mt / col (pristine wave_backward.py:1747-1853, 2320-2327) and the glue's
 * bucket reductions (kbench/api/_implicit_grad.py:288-296).
 */
int kb_rows_sum_accum(int32_t dtype, int32_t S, int32_t m, const int64_t* n, const int32_t* k, const void* const* a,
                      void* const* dst, double* work, void* stream);

/* ---- forward tangents (JVP) of the forward maps, for the Newton HVP path ---- */

/*
 * e_tangent_fixed_point (kbench/core/kernels/e_step_tangent.py:174-208,
 * kernel _e_step_tangent_2d_kernel 27-125): Richardson solve of
 * (I - J_E^EE) dE = J_E^Ep dp at the frozen fixed point E of G item rows,
 * from dE0 (nullable: 0), until max|dE_new - dE| <= tol * max(1, max|dE_new|)
 * or max_iter steps, then dE_s1 / dE_s2 / dEbar of the final dE.  All
 * parameter tensors are [G, S] item-state matrices.  The stopping test is
 * applied per item row (the reference applies it to the max over rows; the
 * two agree for G = 1).  n_iter [G] (nullable) gets the step count.
 * Float32 rows too long for three float64 LDS rows are iterated in float32
 * arithmetic, with tol floored at 8 float32 epsilons (9.5e-7).
 */
typedef struct kb_etan_io {
  int32_t dtype, G, use_col_weights, max_iter;
  double tol;
  const void* E;                                             /* [G, S] */
  const void *log_pS, *log_pD, *log_pL, *max_coupling;       /* [G, S] */
  const void* col_log_probs;                                 /* [S] */
  const void *dlog_pS, *dlog_pD, *dlog_pL, *dmax_coupling;   /* [G, S] */
  const void* dE0;                                           /* [G, S] or NULL */
  void *dE, *dE_s1, *dE_s2, *dEbar;                          /* [G, S] */
  int32_t* n_iter;                                           /* [G] or NULL */
} kb_etan_io;
int kb_e_tangent_fixed_point(const kb_tree* tree, const kb_etan_io* io, void* stream);

/*
 * compute_dts_tangent (kbench/core/kernels/dts_tangent.py:96-122, kernel
 * _dts_tangent_kernel 25-93): out[w, s] = sum over the splits of row w of
 * sum_k 2^(t_k - dts_r[w, s]) dt_k for the five DTL split terms, 0 where
 * dts_r is -inf.  Same split grouping and parameter indexing as
 * kb_dts_forward; the reference's atomic scatter is a fixed-order sum here.
 */
typedef struct kb_dts_tan_io {
  int32_t dtype, S, W, param_by_state;
  int64_t N, item_offset, param_row_stride;
  const int64_t *node_child1, *node_child2;                  /* [S] */
  const void *Pi, *Pibar, *dPi, *dPibar;                     /* [C, S] */
  const int64_t *sl, *sr;                                    /* [N] */
  const void* log_split_probs;                               /* [N] */
  const int32_t *split_ptr, *split_order;                    /* [W + 1], [N] */
  const void *log_pD, *log_pS, *dlog_pD, *dlog_pS;
  const void* dts_r;                                         /* [W, S] */
  const int64_t* item_idx;                                   /* [C] */
  void* out;                                                 /* [W, S] */
} kb_dts_tan_io;
int kb_dts_tangent(const kb_dts_tan_io* io, void* stream);

/*
 * compute_wave_step_tangent (kbench/core/kernels/wave_tangent.py:346-431,
 * kernel 35-177) with n_iters = 1, and compute_wave_step_tangent_selfloop
 * (wave_tangent.py:346-389, kernel 181-343) with n_iters >= 1 and
 * dPi_in == dPi_out, pi_ws == ws: n_iters tangent sweeps of rows
 * [ws, ws + W) at the frozen primal rows Pi_in[pi_ws + w].  The tangent row
 * starts from dPi_in row pi_ws + w; the result goes to dPi_out row ws + w and
 * the dPibar of the last sweep to dPibar_out row ws + w (nullable).  dts and
 * d_dts ([W, S]) are both given for rows with splits, both NULL otherwise.
 * Constant rows as in kb_wave_step; leaf_logp / dleaf_logp rows item * S.
 */
typedef struct kb_wave_tan_io {
  int32_t dtype, S, W, use_col_weights, use_leaf_index, n_iters;
  int64_t ws, pi_ws, const_stride;
  const void *Pi_in, *dPi_in;                                /* [*, S] */
  void* dPi_out;                                             /* [C, S] */
  void* dPibar_out;                                          /* [C, S] or NULL */
  const void *dts, *d_dts;                                   /* [W, S] or NULL */
  const void *max_coupling, *dMC, *DL, *dDL, *Ebar, *dEbar, *E, *dE, *SL1, *dSL1, *SL2, *dSL2;
  const void* col_log_probs;                                 /* [S] */
  const int64_t* item_idx;                                   /* [C] */
  const int64_t* leaf_state;                                 /* [C] */
  const void *leaf_logp, *dleaf_logp;                        /* [G, S] */
} kb_wave_tan_io;
int kb_wave_step_tangent(const kb_tree* tree, const kb_wave_tan_io* io, void* stream);

/* ---- second-order contractions of the backward maps (exact HVP) ---- */

/*
 * e_step_backward_so (kbench/core/kernels/e_step_so.py:182-220, kernels
 * _e_step_so_prepare_kernel 30-158 and _e_step_so_finalize_kernel 161-179):
 * tangent of the E-step VJP at fixed cotangents (g_new, g_ebar) along
 * (dE, dE_new, dE_s1, dE_s2, dEbar, dlog_pS, dlog_pD, dlog_pL, dcol), the row
 * max frozen.  Writes d_grad_E / pS / pD / pL / mc [G, S] and, per item row,
 * the d_grad_col contribution col_rows [G, S] (the caller sums the rows: the
 * reference's atomic column accumulation).  dcol is NULL for a zero tangent.
 */
typedef struct kb_estep_so_io {
  int32_t dtype, G, use_col_weights;
  const void *E, *E_new, *E_s1, *E_s2, *Ebar, *log_pS, *log_pD, *log_pL;   /* [G, S] */
  const void* col_log_probs;                                             /* [S] */
  const void *g_new, *g_ebar;                                            /* [G, S] */
  const void *dE, *dE_new, *dE_s1, *dE_s2, *dEbar, *dlog_pS, *dlog_pD, *dlog_pL;  /* [G, S] */
  const void* dcol;                                                      /* [S] or NULL */
  void *d_grad_E, *d_grad_pS, *d_grad_pD, *d_grad_pL, *d_grad_mc;        /* [G, S] */
  void* col_rows;                                                        /* [G, S] */
} kb_estep_so_io;
int kb_estep_backward_so(const kb_tree* tree, const kb_estep_so_io* io, void* stream);

/*
 * wave_backward_so (kbench/core/kernels/wave_so.py:246-293, kernel 37-243):
 * tangent of one self-loop J^T application and of the parameter buckets
 * (aw0..aw4, aw345) of wave rows [ws, ws + W) at the fixed adjoint v [W, S],
 * along (dPi, dPibar, the constant tangents, d_dts), the saved
 * pibar_row_max frozen.  d_out[w] = d(A^T v)[w] (+ d_rhs[ws + w] when d_rhs
 * is given: the reference's FOLD_RHS).  Constant rows as in kb_wave_step.
 */
typedef struct kb_wave_so_io {
  int32_t dtype, S, W, use_col_weights, use_leaf_index;
  int64_t ws, const_stride;
  const void *Pi, *dPi, *Pibar, *dPibar;                                 /* [C, S] */
  const void* v;                                                         /* [W, S] */
  const void* pibar_row_max;                                             /* [C] */
  const void *DL, *dDL, *Ebar, *dEbar, *E, *dE, *SL1, *dSL1, *SL2, *dSL2;
  const void* col_log_probs;                                             /* [S] */
  const int64_t *item_idx, *leaf_state;                                  /* [C] */
  const void *leaf_logp, *dleaf_logp;                                    /* [G, S] */
  const void *dts, *d_dts;                                               /* [W, S] or NULL */
  const void* d_rhs;                                                     /* [C, S] or NULL */
  void *d_out, *d_aw0, *d_aw1, *d_aw2, *d_aw345, *d_aw3, *d_aw4;         /* [W, S] */
} kb_wave_so_io;
int kb_wave_backward_so(const kb_tree* tree, const kb_wave_so_io* io, void* stream);

/*
 * dts_backward_so (kbench/core/kernels/dts_so.py:233-303, kernels
 * _dts_split_so_kernel 29-141 and _dts_tree_so_kernel 145-230): tangent of
 * the split-term backward and of its Pibar tree VJP at the fixed adjoint v
 * [W, S] of a wave's N splits, along (dPi, dPibar, dlog_pD, dlog_pS, dmt).
 * Instead of the reference's atomic scatters it writes rows the caller adds
 * in a fixed order: side_rows [2N, S] (rows 0..N-1 into Pi rows sl, N..2N-1
 * into sr), col_rows [2N, S] (d_grad_col), pD_rows / pS_rows / mt_rows
 * [N, S] (in the parent row's item).  ud / dud [2N, S] are staging buffers.
 * Rates as in kb_dts_forward; mt / dmt rows item * mt_row_stride.
 */
typedef struct kb_dts_so_io {
  int32_t dtype, S, param_by_state, use_col_weights;
  int64_t N, ws, item_offset, param_row_stride, mt_row_stride;
  const void *Pi, *dPi, *Pibar, *dPibar;                                 /* [C, S] */
  const void* v;                                                         /* [W, S] */
  const int64_t *sl, *sr, *reduce_idx;                                   /* [N] */
  const void* log_split_probs;                                           /* [N] */
  const void *log_pD, *log_pS, *dlog_pD, *dlog_pS, *mt, *dmt;
  const int64_t* item_idx;                                               /* [C] */
  const void* pibar_row_max;                                             /* [C] */
  const void* col_log_probs;                                             /* [S] */
  const int64_t *node_child1, *node_child2;                              /* [S] */
  void *ud, *dud, *side_rows, *col_rows;                                 /* [2N, S] */
  void *pD_rows, *pS_rows, *mt_rows;                                     /* [N, S] */
} kb_dts_so_io;
int kb_dts_backward_so(const kb_tree* tree, const kb_dts_so_io* io, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KBENCH_OPS_H */
