// Fused forward row kernel: one workgroup per clade row does the split
// reduction (dts) or the leaf initialisation, all pi_iters-1 self-loop sweeps,
// and the final Pibar / row max, with the row resident on chip throughout.
//
// Reference semantics (pristine files):
//  * split term dts_r[s] = LSE over the row's splits and the five DTL terms
//    (dts_fused.py:18-168);
//  * leaf initialisation (wave_step.py:223-310);
//  * one sweep Pi_new = LSE(DL+Pi, Pi+Ebar, Pibar(Pi)+E, SL1+Pi[c1], SL2+Pi[c2],
//    leaf | dts) with Pibar(Pi)[s] = log2(sum_{j not anc(s)} 2^Pi_j) + mt
//    (wave_step.py:92-203), run pi_iters-1 times; split rows start from dts_r
//    (forward.py:80-115);
//  * final Pibar and row max from the last Pi (wave_step.py:205-220).
//
// The sweeps run in linear space: x = 2^(Pi - M) with a per-row exponent M
// renormalised by an exact power of two after every sweep (the row sum is
// brought into [1/2, 1)), so a sweep is
//   y = a x + emc NA(x) + k1 x[c1] + k2 x[c2] + (leaf | dts) 2^-M
// with per-position constants a = 2^DL + 2^Ebar, emc = 2^(E+mt), k1 = 2^SL1,
// k2 = 2^SL2 prepared once per solve.  NA(x)[s] = rowsum - pathsum(s) as in
// the reference; the path sums come from an Euler-tour prefix scan.
// Threads own contiguous preorder positions (see kb_rowops.hpp): three
// barriers per sweep.
#include "kb_device.hpp"
#include "kb_kernels.hpp"
#include "kb_rowops.hpp"

namespace kb {

template <int NT, int CPT, bool WEIGHTED>
__global__ __launch_bounds__(NT, (NT == 1024 && CPT == 2) ? 8 : 1) void fwd_row_kernel(FwdParams P, int first) {
  constexpr int MAXS = NT * CPT;
  constexpr int NW = NT / 64;
  __shared__ float Xs[2][MAXS + 64];   // unnormalised y of the sweep (double buffer); [MAXS] == 0
  __shared__ float Sc[2 * MAXS];       // Euler scan / staging
  __shared__ float wtA[NW], wtB[NW];

  const PreDev& T = P.pre;
  const int S = P.S;
  const int tid = threadIdx.x;
  const int row = P.sched_rows[first + blockIdx.x];
  const int leaf_row = P.row_kind[row];
  const int item = P.item[row];
  const size_t cb = (size_t)item * P.const_stride;   // constants are [G, S] in preorder

  OwnTables<NT, CPT> O;
  O.load(T);
  if (tid < 64) {
    Xs[0][MAXS + tid] = 0.0f;
    Xs[1][MAXS + tid] = 0.0f;
  }
  const int(&c1p)[CPT] = O.c1p;
  const int(&c2p)[CPT] = O.c2p;

  // ---- initial row (log2), own positions
  float v[CPT];
  int lpos = -1;
  float leaf_obs = 0.0f;
  if (leaf_row) {
    const int leaf = P.leaf_state[row];
    lpos = T.pre[leaf];
    const int lend = T.endpos[lpos];
    leaf_obs = P.leaf_logp[cb + lpos];
    const float leaf_col = WEIGHTED ? P.col[lpos] : 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = own_pos<NT, CPT>(k);
      v[k] = KB_NEG_INF;
      if (i < S) {
        const bool hit = i == lpos;
        const bool desc = i >= lpos && i < lend;
        const size_t ci = cb + i;
        const float pi_w = hit ? leaf_obs : KB_NEG_INF;
        const float pibar_w = desc ? KB_NEG_INF : P.mt[ci] + leaf_col + leaf_obs;
        const float pi_s1 = c1p[k] == lpos ? leaf_obs : KB_NEG_INF;
        const float pi_s2 = c2p[k] == lpos ? leaf_obs : KB_NEG_INF;  // padding ZERO never equals lpos
        const float t0 = P.DL[ci] + pi_w;
        const float t1 = pi_w + P.Ebar[ci];
        const float t2 = pibar_w + P.E[ci];
        const float t3 = P.SL1[ci] + pi_s1;
        const float t4 = P.SL2[ci] + pi_s2;
        const float t5 = hit ? P.leaf_logp[ci] : KB_NEG_INF;
        const float m = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), fmaxf(t4, t5));
        const float ms = fsafe(m);
        const float sum = exp2f(t0 - ms) + exp2f(t1 - ms) + exp2f(t2 - ms) + exp2f(t3 - ms) + exp2f(t4 - ms) +
                          exp2f(t5 - ms);
        v[k] = log2f(sum) + m;
      }
    }
  } else {
    // child rows staged through LDS at preorder positions (coalesced global
    // loads of column s = tid + j*NT; positions of the padding slot stay 0)
    float* L0 = Xs[0];
    float* L1 = Xs[1];
    float* L2 = Sc;
    float* L3 = Sc + MAXS;
    float m[CPT], acc[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      m[k] = KB_NEG_INF;
      acc[k] = 0.0f;
    }
    const int b = P.split_ptr[row], e = P.split_ptr[row + 1];
    for (int si = b; si < e; ++si) {
      const size_t l = (size_t)P.split_l[si] * S, r = (size_t)P.split_r[si] * S;
      const float lsp = P.split_lsp[si];
      if (si > b) __syncthreads();  // the previous split's readers are done
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        const int sj = tid + j * NT;
        if (sj < S) {
          const int i = T.pre[sj];
          L0[i] = P.pi[l + sj];
          L1[i] = P.pi[r + sj];
          L2[i] = P.pibar[l + sj];
          L3[i] = P.pibar[r + sj];
        }
      }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int i = own_pos<NT, CPT>(k);
        if (i < S) {
          const bool h1 = c1p[k] != MAXS, h2 = c2p[k] != MAXS;
          const float pl = L0[i], pr = L1[i];
          const float d = P.pD.at(item, i), sp = P.pS.at(item, i);
          const float t0 = lsp + d + pl + pr;
          const float t1 = lsp + pl + L3[i];
          const float t2 = lsp + pr + L2[i];
          const float l1 = h1 ? L0[c1p[k]] : KB_NEG_INF, r1 = h1 ? L1[c1p[k]] : KB_NEG_INF;
          const float l2 = h2 ? L0[c2p[k]] : KB_NEG_INF, r2 = h2 ? L1[c2p[k]] : KB_NEG_INF;
          const float t3 = lsp + sp + l1 + r2;
          const float t4 = lsp + sp + r1 + l2;
          const float m5 = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), t4);
          const float ms = fsafe(m5);
          const float s5 = exp2f(t0 - ms) + exp2f(t1 - ms) + exp2f(t2 - ms) + exp2f(t3 - ms) + exp2f(t4 - ms);
          lse_merge(m[k], acc[k], m5, s5);
        }
      }
    }
    __syncthreads();  // the staging buffers become the sweep buffers
#pragma unroll
    for (int k = 0; k < CPT; ++k) v[k] = log2f(acc[k]) + m[k];
    if (P.dts_out) {  // the backward reuses the split term at Pi*
      float* dst = P.dts_out + (size_t)row * S;
#pragma unroll
      for (int k = 0; k < CPT; ++k)
        if (own_pos<NT, CPT>(k) < S) dst[own_pos<NT, CPT>(k)] = v[k];
    }
  }

  // ---- linear space relative to the row maximum
  float lm = KB_NEG_INF;
#pragma unroll
  for (int k = 0; k < CPT; ++k) lm = fmaxf(lm, v[k]);
  const float Ms = fsafe(block_max1<NT>(lm, wtB));  // wtA is written next without a barrier
  float y[CPT], dl[CPT], ca[CPT], ce[CPT], ck1[CPT], ck2[CPT], cw[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = own_pos<NT, CPT>(k);
    const bool ok = i < S;
    y[k] = ok ? exp2f(v[k] - Ms) : 0.0f;
    dl[k] = leaf_row ? 0.0f : y[k];
    ca[k] = ok ? P.lin_a[cb + i] : 0.0f;
    ce[k] = ok ? P.lin_emc[cb + i] : 0.0f;
    ck1[k] = ok ? P.lin_k1[cb + i] : 0.0f;
    ck2[k] = ok ? P.lin_k2[cb + i] : 0.0f;
    cw[k] = WEIGHTED ? (ok ? P.colw[i] : 0.0f) : 1.0f;
  }
  const float leaf_lin = leaf_row ? exp2f(leaf_obs - Ms) : 0.0f;  // lpos = -1 for split rows
  int kexp = 0;
  float x[CPT], ps[CPT], rowsum = 0.0f, f = 1.0f;

  for (int sweep = 0;; ++sweep) {
    float* X = Xs[sweep & 1];
    // phase A: publish y (padding slot stays 0), reduce the (weighted) row sum,
    // renormalise by an exact power of two
    float ls = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      X[own_pos<NT, CPT>(k)] = y[k];
      ls += cw[k] * y[k];
    }
    const float tsum = block_sum1<NT>(ls, wtA);
    const int e = tsum > 0.0f ? __builtin_amdgcn_frexp_expf(tsum) : 0;
    f = __builtin_amdgcn_ldexpf(1.0f, -e);
    kexp += e;
    rowsum = tsum * f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) x[k] = y[k] * f;
    // ancestors-or-self path sums (of the unnormalised values)
    path_sum_euler<NT, CPT>(O, X, Sc, wtB, ps, WEIGHTED ? P.colw : nullptr);
    if (sweep == P.n_sweeps) break;
    const float scale = __builtin_amdgcn_ldexpf(1.0f, -kexp);
    const float lterm = leaf_lin * scale;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const float na = fmaxf(rowsum - ps[k] * f, 0.0f);
      float yy = ca[k] * x[k] + ce[k] * na;
      yy += ck1[k] * (X[c1p[k]] * f);
      yy += ck2[k] * (X[c2p[k]] * f);
      yy += dl[k] * scale;
      yy += own_pos<NT, CPT>(k) == lpos ? lterm : 0.0f;
      y[k] = yy;
    }
  }

  // ---- outputs: Pi, Pibar from the final Pi, and the (weighted) row max
  const float M = Ms + (float)kexp;
  float piv[CPT], pbv[CPT];
  float lmax = KB_NEG_INF;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = own_pos<NT, CPT>(k);
    piv[k] = KB_NEG_INF;
    pbv[k] = KB_NEG_INF;
    if (i < S) {
      piv[k] = x[k] > 0.0f ? log2f(x[k]) + M : KB_NEG_INF;
      const float na = rowsum - ps[k] * f;
      pbv[k] = na > 0.0f ? log2f(na) + M + P.mt[cb + i] : KB_NEG_INF;
      lmax = fmaxf(lmax, WEIGHTED ? P.col[i] + piv[k] : piv[k]);
    }
  }
  // Sc (last read inside path_sum_euler) is reused as staging after this barrier.
  const float rmax = block_max1<NT>(lmax, wtA);
  const size_t rb = (size_t)row * S;
  store_row_pre<NT, CPT>(T, piv, Sc, P.pi + rb);
  store_row_pre<NT, CPT>(T, pbv, Sc + MAXS, P.pibar + rb);
  if (tid == 0) P.rowmax[row] = rmax;
}

#define KB_FWD_CASE(NT_, CPT_)                                                                            \
  if (S <= NT_ * CPT_) {                                                                                  \
    if (P.use_col)                                                                                        \
      hipLaunchKernelGGL((fwd_row_kernel<NT_, CPT_, true>), dim3(W), dim3(NT_), 0, st, P, first);         \
    else                                                                                                  \
      hipLaunchKernelGGL((fwd_row_kernel<NT_, CPT_, false>), dim3(W), dim3(NT_), 0, st, P, first);        \
    return;                                                                                               \
  }

// One workgroup per copied row (rows of a class are identical).
__global__ __launch_bounds__(256) void copy_rows_kernel(float* pi, float* pibar, float* rowmax, const int* dst,
                                                        const int* src, int S) {
  const size_t d = (size_t)dst[blockIdx.x] * S, s = (size_t)src[blockIdx.x] * S;
  for (int j0 = threadIdx.x; j0 < S; j0 += 4 * 256) {  // 8 independent loads in flight per thread
    float a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + u * 256;
      a[u] = j < S ? pi[s + j] : 0.0f;
      b[u] = j < S ? pibar[s + j] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + u * 256;
      if (j < S) {
        pi[d + j] = a[u];
        pibar[d + j] = b[u];
      }
    }
  }
  if (threadIdx.x == 0) rowmax[dst[blockIdx.x]] = rowmax[src[blockIdx.x]];
}

void launch_copy_rows(float* pi, float* pibar, float* rowmax, const int* dst, const int* src, int n, int S,
                      hipStream_t st) {
  if (n <= 0) return;
  hipLaunchKernelGGL(copy_rows_kernel, dim3(n), dim3(256), 0, st, pi, pibar, rowmax, dst, src, S);
}

void launch_fwd_wave(const FwdParams& P, int first, int W, hipStream_t st) {
  if (W <= 0) return;
  const int S = P.S;
  if (P.wide == 1) {  // fewer, wider threads per row (tuning knob)
    KB_FWD_CASE(256, 8)
  }
  if (P.wide == 2) {  // more, narrower threads per row (tuning knob)
    KB_FWD_CASE(1024, 2)
  }
  KB_FWD_CASE(64, 2)
  KB_FWD_CASE(128, 2)
  KB_FWD_CASE(256, 2)
  KB_FWD_CASE(256, 4)
  KB_FWD_CASE(512, 4)
  KB_FWD_CASE(1024, 4)
  KB_FWD_CASE(1024, 8)
}

}  // namespace kb
