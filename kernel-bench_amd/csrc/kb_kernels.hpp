// Kernel parameter blocks and launchers shared between the kernel sources and
// the C-ABI layer (kb_api.hip).
#pragma once

#include "kb_device.hpp"

namespace kb {

// ----------------------------------------------------------------------------
// parameters + E-step (kb_estep.hip)
// ----------------------------------------------------------------------------
struct EStepParams {
  TreeDev tr;
  int S;
  int n_tlevels;              // depth levels, root first
  const int* tlevel_ptr;      // [n_tlevels + 1]
  const int* tlevel_node;     // [S]
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
  // per-column constants of the wave kernels (float32, [S])
  float* c_DL; float* c_SL1; float* c_SL2; float* c_pS; float* c_pD; float* c_colw;
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
  int S;
  int n_sweeps;               // pi_iters - 1
  int use_col;
  int const_stride;           // 0: one constant row; S: item-indexed rows
  // per-column constants, row = item * const_stride
  const float* lin_a; const float* lin_emc; const float* lin_k1; const float* lin_k2;
  const float* colw;          // [S] 2^col_log_probs (weighted) -- may be null when !use_col
  const float* col;           // [S]
  const float* mt; const float* DL; const float* Ebar; const float* E; const float* SL1; const float* SL2;
  const float* leaf_logp;     // [G,S] log pS used by the leaf term
  RateDev pD, pS;             // split-term rates
  // layout
  const int* item;            // [C]
  const int* leaf_state;      // [C]
  const int* split_ptr;       // [C+1] splits of each parent row
  const int* split_l; const int* split_r; const float* split_lsp;
  // outputs
  float* pi; float* pibar; float* rowmax;
};

void launch_fwd_wave(const FwdParams& P, int ws, int W, int leaf_wave, hipStream_t st);

}  // namespace kb
