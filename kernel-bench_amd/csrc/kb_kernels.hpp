// Kernel parameter blocks and launchers shared between the kernel sources and
// the C-ABI layer (kb_api.hip).
#pragma once

#include "kb_device.hpp"
#include "kb_rowops.hpp"

namespace kb {

// Records the message returned by kb_last_error(); returns `code`.
int set_error(int code, const char* fmt, ...);


// ----------------------------------------------------------------------------
// parameters + E-step (kb_estep.hip)
// ----------------------------------------------------------------------------
struct EStepParams {
  TreeDev tr;
  TreeScanDev ts;
  PreDev pd;                  // preorder tables (register-resident kernel)
  int S;
  int n_tlevels;              // depth levels, root first
  const int* tlevel_ptr;      // [n_tlevels + 1]
  const int* tlevel_node;     // [S]
  const int* pre;             // [S] column -> preorder position (layout of the c_* / lin_* constants)
  const float* theta;         // [S,3] (statewise) or [3]
  int statewise;
  const float* col_weights;   // [S]
  int use_col;
  const float* unnorm_row_max;  // [S]
  double e_init;
  int max_iter;
  double tol;
  // saved forward outputs (float32)
  float* E; float* E_s1; float* E_s2; float* Ebar;
  float* log_pS; float* log_pD; float* log_pL;   // [S] statewise, [1] global
  float* mt; float* col_log_probs;               // [S]
  double* E64;                                    // optional float64 E
  int* n_iter_out;
  // constants of the row kernels (float32, [S], preorder positions)
  float* c_DL; float* c_SL1; float* c_SL2; float* c_pS; float* c_pD; float* c_colw;
  float* c_Ebar; float* c_E; float* c_mt; float* c_col;
  float* lin_a; float* lin_emc; float* lin_k1; float* lin_k2;
};

void launch_estep(const EStepParams& P, hipStream_t st);
void launch_loss(const float* pi, const int* root_rows, const float* E, int S, int n_fam, double* terms,
                 double* loss64, float* loss32, hipStream_t st);

// ----------------------------------------------------------------------------
// forward wave kernels (kb_fwd.hip)
// ----------------------------------------------------------------------------
struct FwdParams {
  TreeDev tr;
  PreDev pre;
  int S;
  int wide;                   // 1: 256 x 8, 2: 1024 x 2 on every level, 3: no narrow shape
  int narrow_below;           // wide == 0: 1024 x 2 on levels with fewer rows than this (and the leaf level)
  int n_sweeps;               // pi_iters - 1
  int use_col;
  // per-position constants: one [S] row in preorder, shared by every row
  const float* lin_a; const float* lin_emc; const float* lin_k1; const float* lin_k2;
  const float* colw;          // [S] 2^col_log_probs (weighted) -- may be null when !use_col
  const float* col;           // [S]
  const float* mt; const float* DL; const float* Ebar; const float* E; const float* SL1; const float* SL2;
  const float* pD; const float* pS;  // [S] split-term rates (pS is also the leaf term's log pS)
  // layout
  const int* leaf_state;      // [C]
  const int* split_ptr;       // [C+1] splits of each parent row
  const int* split_l; const int* split_r; const float* split_lsp;
  const int* sched_rows;      // rows in dependency-level order
  const int* row_kind;        // 1: leaf row, 0: split row
  const int* dup_ptr;         // [slots + 1] rows identical to the row of each slot ...
  const int* dup_rows;        // ... which receive the same outputs
  const int* om_tab;          // owner-major position tables (OmTab) for rows of 4097..8192 states, or null
  int large;                  // 1: rows of 4097..8192 states run fwd_row_kernel on om_tab (else the Euler kernel)
  // outputs
  float* pi; float* pibar; float* rowmax;
  float* dts_out;             // [C, S] preorder split term of every computed split row
};

// Pi / Pibar / row-max rows src[i] -> dst[i], i < n.
// Launch the rows sched_rows[first .. first + n).
void launch_fwd_wave(const FwdParams& P, int first, int n, hipStream_t st);

// ----------------------------------------------------------------------------
// backward (kb_bwd.hip, kb_epi.hip)
// ----------------------------------------------------------------------------
struct BwdConstArgs {
  int S;
  int statewise;
  const int* pre;
  const float* log_pS; const float* log_pD; const float* E; const float* E_s1; const float* E_s2;
  const float* Ebar; const float* mt; const float* col;
  // outputs at preorder positions
  float* DL; float* SL1; float* SL2; float* pS_state; float* pD_state;
  float* Ebar_pre; float* E_pre; float* mt_pre; float* col_pre;
  float* om;                  // also in the owner-major layout (KB_OM_CONSTS rows), or null
  float* zero; size_t n_zero;  // n_zero floats set to zero by the same launch (the bucket slots)
};

// Owner-major layout of bwd_row_large_kernel's per-position tables: with
// 1024 threads owning CPT positions each (thread t: t*CPT .. t*CPT+CPT-1),
// row j holds position t*CPT + k at [j*1024*CPT + k*1024 + t], so a
// wavefront's reads of one slot k are contiguous.
enum OmConst { OMC_DL, OMC_EBAR, OMC_E, OMC_SL1, OMC_SL2, OMC_PD, OMC_PS, OMC_MT, OMC_COL, KB_OM_CONSTS };
// position tables: child-1 / child-2 positions (-1: leaf); parent position
// (ZERO = 1024*CPT for the root) | (subtree end - 1) << 16 | child-1 flag << 30;
// postorder slot's position | (tin(i) - i) << 16.  Positions >= S: -1, -1,
// ZERO | ZERO << 16, ZERO.
enum OmTab { OMT_C1, OMT_C2, OMT_PK, OMT_PN, KB_OM_TABS };

// The backward's record of a schedule slot (KB_BREC ints): the row's first
// two child sides (-1: none; bit 30 of the second: more sides follow), the
// row, its family root index (-1: not a root), leaf-row flag, split range,
// class representative, the first split's children (-1: no split) and log
// split probability (float bits), and the leaf's preorder position (-1: split
// row).
enum BrecField {
  BR_S0, BR_S1, BR_ROW, BR_FAM, BR_LEAF, BR_SB, BR_SE, BR_REP, BR_L0, BR_R0, BR_LSP0, BR_LPOS,
  KB_BREC = 16
};

struct BwdParams {
  TreeDev tr;
  PreDev pre;
  int S;
  int n_terms;                // neumann_terms
  float rtol;                 // > 0: the series stops at the first term below rtol * max|rhs| (0: all terms)
  unsigned char* terms_out;   // optional [C]: J^T applications of each solved row
  float thr;                  // adjoint_pruning_threshold
  int use_pruning;
  int use_col;
  // per-position constants: one [S] row in preorder, shared by every row
  const float* DL; const float* Ebar; const float* E; const float* SL1; const float* SL2;
  const float* mt; const float* col;
  const float* pD; const float* pS;  // [S] split-term rates (pS is also the leaf term's log pS)
  const float* pi; const float* pibar; const float* rowmax;
  const int* leaf_state; const int* root_index;
  const int* split_ptr; const int* split_l; const int* split_r; const float* split_lsp;
  const int* child_ptr; const int* child_in;
  const int* bslot;           // [KB_BREC * C] record of every schedule slot (BrecField)
  float* staging;             // [2 * n_splits, kb_stage_ld(S)]
  unsigned char* split_on;    // [n_splits]
  unsigned char* mask;        // [C]
  float* contrib;             // [n_partials, 8, kb_slot_ld(S)] gradient buckets, one slot per workgroup
  const int* sched_rows;
  const int* row_kind;
  int class_mode;             // 1: entries are classes of identical rows (cls_ptr / cls_rows)
  int variant;                // launch shape: 0 default, 2 narrow (1024 threads x 2 states)
  int large;                  // 1: rows of 2049..8192 states run bwd_row_large_kernel
  const int* om_tab;          // [KB_OM_TABS, kb_large_ld(S)] owner-major position tables (OmTab)
  const float* om_const;      // [KB_OM_CONSTS, kb_large_ld(S)] owner-major constants (OmConst)
  float* rhs0;                // [rows of level 0, S] preorder adjoint rows, in cls_rows order
  float* rhsc;                // [classes of level 0, S] summed adjoint of each class
  const int* m_side_ptr;      // [members + 1] staging sides of each level-0 member (cls_rows order)
  const int* m_side;
  const int* m_root;          // [members] family of a member that is a root row, else -1
  unsigned char* m_mask;      // [members] active mask in member order
  unsigned char* cls_active;  // [classes of level 0] any member active
  const float* dts_in;        // [C, S] preorder split terms stored by the forward, or null: recompute
  const int* rep_of;          // [C] row -> row whose stored split term it shares
  const int* cls_ptr;         // [n_classes + 1]
  const int* cls_rows;        // member rows, representative first
  // level-0 classes cut into chunks of at most KB_CHUNK0 members
  int n_chunks0;
  const int* ck_ptr;          // [chunks + 1] member (cls_rows) ranges
  const int* cls_ck_ptr;      // [classes + 1] chunk ranges
  unsigned char* ck_any;      // [chunks] any member of the chunk active
};

constexpr int KB_CHUNK0 = 8;
// Workgroup slot of bwd_row_large_kernel: KB_LARGE_SLOT_ROWS rows of
// kb_large_ld(S) floats (8 bucket rows, then the row's split term, Pi* and
// Pibar*); other row kernels use 8 rows of kb_slot_ld(S).
constexpr int KB_LARGE_SLOT_ROWS = 11;
// large = 1: rows of 2049..8192 states; large = 2: also rows of 1025..2048
// states (512 threads x 4 positions)
__host__ __device__ inline bool kb_use_large(int S, int large) {
  return (large && S > 2048 && S <= 8192) || (large == 2 && S > 1024 && S <= 2048);
}
// threads and positions (owner-major row length) of the low-register kernel's shape for S states
__host__ __device__ inline int kb_large_nt(int S) { return S <= 2048 ? 512 : 1024; }
__host__ __device__ inline int kb_large_ld(int S) { return S <= 2048 ? 2048 : (S <= 4096 ? 4096 : 8192); }
// row stride (floats) of the workgroup bucket slots: kb_large_ld for the
// low-register kernel, else S rounded up to a multiple of four (16-byte rows)
// row stride (floats) of the backward's child staging rows: S rounded up to a
// multiple of four, so rows start 16-byte aligned.  The allocation ends with
// KB_STAGE_TAIL more floats, so a row kernel's vector read of its own positions
// (up to 2048 from a row's start) stays inside it for every row.
__host__ __device__ inline int kb_stage_ld(int S) { return (S + 3) & ~3; }
constexpr int KB_STAGE_TAIL = 2048;
__host__ __device__ inline int kb_slot_ld(int S, int large) {
  return kb_use_large(S, large) ? kb_large_ld(S) : ((S + 3) & ~3);
}

struct EpiParams {
  TreeDev tr;
  TreeScanDev ts;
  PreDev pd;                  // preorder tables (register-resident kernel)
  int S;
  int n_tlevels;
  const int* tlevel_ptr;
  const int* tlevel_node;
  const float* E; const float* log_pS; const float* log_pD; const float* log_pL; const float* mt;
  const float* col;
  int statewise;
  int use_col;
  const float* theta;
  const float* col_weights;
  const double* acc;          // [8, S]
  int n_fam;
  int n_items_rows;           // rows of E (1 unless itemwise)
  int max_iter;
  double tol;
  double breakdown;
  float* grad_theta;
  float* grad_col;
  double* work;               // [N_WORK, S]
  int* status;                // [0] iterations, [1] failure flag
  const double* q_extra;      // [S] added to q_E, or null
  int no_norm;                // 1: q_E without the loss normaliser's term
  double* w_out;              // [S] E adjoint out (with g_out), or null
  double* g_out;              // [5, S] cotangents of (pS, pD, pL, mt, col) per state; when set the
                              // kernel ends after them (no theta / column VJP)
};

void launch_bwd_consts(const BwdConstArgs& A, hipStream_t st);
// Rows sched_rows[first .. first + n) on nb workgroups (round-robin); partial
// bucket rows poff .. poff + nb.
void launch_bwd_wave(const BwdParams& P, int first, int n, int nb, int poff, hipStream_t st);
int bwd_blocks_per_cu(int S, int use_col, int variant, int large);
// Rows of 2049..8192 states on the low-register kernel (kb_bwd_large.hip);
// false if P.large is off or S is outside that range.
bool launch_bwd_large(const BwdParams& P, int first, int n, int nb, int poff, hipStream_t st);
int bwd_large_blocks_per_cu(int S, int use_col);
// Level-0 adjoint rows, masks and class sums.
void launch_bwd_level0_prep(const BwdParams& P, int n_members, int n_cls, hipStream_t st);
// Sums the bucket rows of C workgroup slots (slot_stride floats apart, bucket
// rows ld floats apart, preorder positions) in slot order into out [8, S] in
// column order (column s at preorder position pre[s]).
void launch_bwd_reduce(const float* contrib, int C, int S, size_t slot_stride, int ld, double* partial, const int* pre,
                       double* out, hipStream_t st);
int reduce_chunks(int C);
void launch_epilogue(const EpiParams& P, hipStream_t st);
int epilogue_work_vectors();

}  // namespace kb
