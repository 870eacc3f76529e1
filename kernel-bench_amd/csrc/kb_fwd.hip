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
// Two layouts of the sweep loop:
//  * fwd_row_kernel (rows of up to 8192 positions; 8 per thread with the
//    owner-major tables): two barriers per sweep.  Thread t owns preorder
//    positions t*CPT+k and postorder slots t*CPT+k.  The path sum is
//    ps(i) = Pre(i) - PostEx(tin(i) - i),  Pre the inclusive preorder prefix
//    sum and PostEx the exclusive postorder prefix sum (the nodes left before
//    entering i, tin(i) - i of them, are the first ones in postorder).  Phase
//    A scans the own positions in registers and publishes y and the
//    wavefront totals; after the first barrier each thread reads the values
//    of its postorder slots and scans them (phase B), published under the
//    second barrier; phase C forms the path sums, the wavefront offsets being
//    applied by the readers.
//  * fwd_row_kernel_euler (rows past 4096 positions without the owner-major
//    tables): wavefront-segment ownership and an Euler-tour scan, three
//    barriers per sweep, half the LDS.
#include "kb_device.hpp"
#include "kb_kernels.hpp"
#include "kb_rowops.hpp"

namespace kb {

template <int NT, int CPT, bool WEIGHTED>
__global__ __launch_bounds__(NT, (NT == 1024 && CPT == 2) ? 8 : 1) void fwd_row_kernel_euler(FwdParams P, int first) {
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
    leaf_obs = P.pS[lpos];
    const float leaf_col = WEIGHTED ? P.col[lpos] : 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = own_pos<NT, CPT>(k);
      v[k] = KB_NEG_INF;
      if (i < S) {
        const bool hit = i == lpos;
        const bool desc = i >= lpos && i < lend;
        const int ci = i;
        const float pi_w = hit ? leaf_obs : KB_NEG_INF;
        const float pibar_w = desc ? KB_NEG_INF : P.mt[ci] + leaf_col + leaf_obs;
        const float pi_s1 = c1p[k] == lpos ? leaf_obs : KB_NEG_INF;
        const float pi_s2 = c2p[k] == lpos ? leaf_obs : KB_NEG_INF;  // padding ZERO never equals lpos
        const float t0 = P.DL[ci] + pi_w;
        const float t1 = pi_w + P.Ebar[ci];
        const float t2 = pibar_w + P.E[ci];
        const float t3 = P.SL1[ci] + pi_s1;
        const float t4 = P.SL2[ci] + pi_s2;
        const float t5 = hit ? P.pS[ci] : KB_NEG_INF;
        const float m = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), fmaxf(t4, t5));
        const float ms = fsafe(m);
        const float sum = exp2_hw(t0 - ms) + exp2_hw(t1 - ms) + exp2_hw(t2 - ms) + exp2_hw(t3 - ms) +
                          exp2_hw(t4 - ms) + exp2_hw(t5 - ms);
        v[k] = log2_hw(sum) + m;
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
          const float d = P.pD[i], sp = P.pS[i];
          const float t0 = lsp + d + pl + pr;
          const float t1 = lsp + pl + L3[i];
          const float t2 = lsp + pr + L2[i];
          const float l1 = h1 ? L0[c1p[k]] : KB_NEG_INF, r1 = h1 ? L1[c1p[k]] : KB_NEG_INF;
          const float l2 = h2 ? L0[c2p[k]] : KB_NEG_INF, r2 = h2 ? L1[c2p[k]] : KB_NEG_INF;
          const float t3 = lsp + sp + l1 + r2;
          const float t4 = lsp + sp + r1 + l2;
          const float m5 = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), t4);
          const float ms = fsafe(m5);
          const float s5 =
              exp2_hw(t0 - ms) + exp2_hw(t1 - ms) + exp2_hw(t2 - ms) + exp2_hw(t3 - ms) + exp2_hw(t4 - ms);
          lse_merge(m[k], acc[k], m5, s5);
        }
      }
    }
    __syncthreads();  // the staging buffers become the sweep buffers
#pragma unroll
    for (int k = 0; k < CPT; ++k) v[k] = log2_hw(acc[k]) + m[k];
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
    ca[k] = ok ? P.lin_a[i] : 0.0f;
    ce[k] = ok ? P.lin_emc[i] : 0.0f;
    ck1[k] = ok ? P.lin_k1[i] : 0.0f;
    ck2[k] = ok ? P.lin_k2[i] : 0.0f;
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
      pbv[k] = na > 0.0f ? log2f(na) + M + P.mt[i] : KB_NEG_INF;
      lmax = fmaxf(lmax, WEIGHTED ? P.col[i] + piv[k] : piv[k]);
    }
  }
  // Sc (last read inside path_sum_euler) is reused as staging after this barrier.
  const float rmax = block_max1<NT>(lmax, wtA);
  const size_t rb = (size_t)row * S;
  store_row_pre<NT, CPT>(T, piv, Sc, P.pi + rb);
  store_row_pre<NT, CPT>(T, pbv, Sc + MAXS, P.pibar + rb);
  if (tid == 0) P.rowmax[row] = rmax;
  // the rows identical to this one get the same outputs (still staged in Sc)
  for (int d = P.dup_ptr[first + blockIdx.x]; d < P.dup_ptr[first + blockIdx.x + 1]; ++d) {
    const int r2 = P.dup_rows[d];
    const size_t b2 = (size_t)r2 * S;
    for (int s = tid; s < S; s += NT) {
      const int i = T.pre[s];
      P.pi[b2 + s] = Sc[i];
      P.pibar[b2 + s] = Sc[MAXS + i];
    }
    if (tid == 0) P.rowmax[r2] = rmax;
  }
}

// Minimum waves per SIMD (the second launch-bounds argument): 6 keeps three
// 512 x 4 workgroups resident per CU (at most 80 VGPRs; the weighted variant
// would spill).
#define FWD_MIN_WAVES(NT, CPT, W) (((NT) == 512 && (CPT) == 4 && !(W)) ? 6 : 1)

template <int NT, int CPT, bool WEIGHTED>
__global__ __launch_bounds__(NT, FWD_MIN_WAVES(NT, CPT, WEIGHTED)) void fwd_row_kernel(FwdParams P, int first) {
  constexpr int MAXS = NT * CPT;
  constexpr int NW = NT / 64;
  constexpr int ZERO = MAXS;      // padding slot: 0 in the sweep buffers
  constexpr int SEG = 64 * CPT;   // postorder slots per wavefront
  __shared__ __align__(16) float Lb[4][MAXS + 64];  // split staging; then X (y of the sweep), Q (postorder scan)
  __shared__ float wP[NW], wQ[NW], wM[NW];
  float* X = Lb[0];
  float* Q = Lb[1];

  const PreDev& T = P.pre;
  const int S = P.S;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int row = P.sched_rows[first + blockIdx.x];
  const int leaf_row = P.row_kind[row];

  // Tables of the own positions i = tid*CPT + k and of the own postorder slots.
  // In preorder (child1 first) child1 of i is i + 1: from registers, except
  // for the last own position, whose child1 is read from X.  With 8 positions
  // per thread (and the owner-major tables given) the sweeps read child2, the
  // postorder slot and tin(i) - i from those tables in every sweep instead of
  // holding them in registers.
  constexpr bool OMT = CPT == 8;
  int c2p[CPT], nex[CPT], qp[CPT], pre_s[CPT];
  bool h1[CPT];
  // Below 1024 threads the tables and row constants are read with one vector
  // load per row (they start their allocations); the 1024 x 2 shape keeps one
  // load per position, which measured faster there.
  constexpr bool VEC = NT < 1024;
  if constexpr (VEC) {
    int a[CPT], tn[CPT];
    gld_own<CPT>(T.c1pos, S, a, -1);
    gld_own<CPT>(T.c2pos, S, c2p, -1);
    gld_own<CPT>(T.tin, S, tn, 0);
    gld_own<CPT>(T.post, S, qp, ZERO);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = own_pos_c<NT, CPT>(k);
      h1[k] = a[k] >= 0;
      c2p[k] = c2p[k] >= 0 ? c2p[k] : ZERO;
      nex[k] = i < S ? tn[k] - i : 0;
      const int sj = tid + k * NT;
      pre_s[k] = sj < S ? T.pre[sj] : 0;
    }
  } else {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = own_pos_c<NT, CPT>(k);
      const bool ok = i < S;
      const int a = ok ? T.c1pos[i] : -1, b = ok ? T.c2pos[i] : -1;
      h1[k] = a >= 0;
      c2p[k] = b >= 0 ? b : ZERO;
      nex[k] = ok ? T.tin[i] - i : 0;
      qp[k] = ok ? T.post[i] : ZERO;
      const int sj = tid + k * NT;
      pre_s[k] = sj < S ? T.pre[sj] : 0;
    }
  }
  const int c1last = h1[CPT - 1] ? own_pos_c<NT, CPT>(CPT - 1) + 1 : ZERO;

  // Per-position row constants.  Shapes of two positions per thread have
  // registers to spare and run the levels with few rows per CU, where a row's
  // dependent loads are not hidden by other workgroups: they load the
  // constants before the row's own loads, so the latencies overlap.
  constexpr bool EARLY = CPT == 2;
  float kd[CPT], ks[CPT], ca[CPT], ce[CPT], ck1[CPT], ck2[CPT];
  auto load_lin = [&]() {
    if constexpr (VEC) {
      gld_own<CPT>(P.lin_a, S, ca, 0.0f);
      gld_own<CPT>(P.lin_emc, S, ce, 0.0f);
      gld_own<CPT>(P.lin_k1, S, ck1, 0.0f);
      gld_own<CPT>(P.lin_k2, S, ck2, 0.0f);
#pragma unroll
      for (int k = 0; k < CPT; ++k) ck1[k] = h1[k] ? ck1[k] : 0.0f;  // 0 without child1: the x1 operand is then unused
    } else {
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int i = own_pos_c<NT, CPT>(k);
        const bool ok = i < S;
        ca[k] = ok ? P.lin_a[i] : 0.0f;
        ce[k] = ok ? P.lin_emc[i] : 0.0f;
        ck1[k] = h1[k] ? P.lin_k1[i] : 0.0f;  // 0 without child1: the x1 operand is then unused
        ck2[k] = ok ? P.lin_k2[i] : 0.0f;
      }
    }
  };
  if constexpr (EARLY) {
    load_lin();
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = own_pos_c<NT, CPT>(k);
      kd[k] = i < S ? P.pD[i] : 0.0f;
      ks[k] = i < S ? P.pS[i] : 0.0f;
    }
  }

  // ---- initial row (log2), own positions
  float v[CPT];
  int lpos = -1;
  float leaf_obs = 0.0f;
  if (leaf_row) {
    const int leaf = P.leaf_state[row];
    lpos = T.pre[leaf];
    const int lend = T.endpos[lpos];
    leaf_obs = P.pS[lpos];
    const float leaf_col = WEIGHTED ? P.col[lpos] : 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = own_pos_c<NT, CPT>(k);
      v[k] = KB_NEG_INF;
      if (i < S) {
        const bool hit = i == lpos;
        const bool desc = i >= lpos && i < lend;
        const int ci = i;
        const float pi_w = hit ? leaf_obs : KB_NEG_INF;
        const float pibar_w = desc ? KB_NEG_INF : P.mt[ci] + leaf_col + leaf_obs;
        const float pi_s1 = (h1[k] && i + 1 == lpos) ? leaf_obs : KB_NEG_INF;
        const float pi_s2 = c2p[k] == lpos ? leaf_obs : KB_NEG_INF;  // padding ZERO never equals lpos
        const float t0 = P.DL[ci] + pi_w;
        const float t1 = pi_w + P.Ebar[ci];
        const float t2 = pibar_w + P.E[ci];
        const float t3 = P.SL1[ci] + pi_s1;
        const float t4 = P.SL2[ci] + pi_s2;
        const float t5 = hit ? P.pS[ci] : KB_NEG_INF;
        const float m = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), fmaxf(t4, t5));
        const float ms = fsafe(m);
        const float sum = exp2_hw(t0 - ms) + exp2_hw(t1 - ms) + exp2_hw(t2 - ms) + exp2_hw(t3 - ms) +
                          exp2_hw(t4 - ms) + exp2_hw(t5 - ms);
        v[k] = log2_hw(sum) + m;
      }
    }
  } else {
    // child rows staged through LDS at preorder positions (coalesced global
    // loads of column s = tid + j*NT)
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
          const int i = pre_s[j];
          Lb[0][i] = P.pi[l + sj];
          Lb[1][i] = P.pi[r + sj];
          Lb[2][i] = P.pibar[l + sj];
          Lb[3][i] = P.pibar[r + sj];
        }
      }
      __syncthreads();
      float pl[CPT], pr[CPT], bl[CPT], br[CPT];
      lds_load_own<CPT>(Lb[0], pl);
      lds_load_own<CPT>(Lb[1], pr);
      lds_load_own<CPT>(Lb[2], bl);
      lds_load_own<CPT>(Lb[3], br);
      const bool hl = h1[CPT - 1];
      const float pl_last = hl ? Lb[0][c1last] : KB_NEG_INF, pr_last = hl ? Lb[1][c1last] : KB_NEG_INF;
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int i = own_pos_c<NT, CPT>(k);
        if (i < S) {
          const bool h2 = c2p[k] != ZERO;
          const float d = EARLY ? kd[k] : P.pD[i], sp = EARLY ? ks[k] : P.pS[i];
          const float t0 = lsp + d + pl[k] + pr[k];
          const float t1 = lsp + pl[k] + br[k];
          const float t2 = lsp + pr[k] + bl[k];
          float l1, r1;
          if (k + 1 < CPT) {
            l1 = h1[k] ? pl[k + 1] : KB_NEG_INF;
            r1 = h1[k] ? pr[k + 1] : KB_NEG_INF;
          } else {
            l1 = pl_last;
            r1 = pr_last;
          }
          const float l2 = h2 ? Lb[0][c2p[k]] : KB_NEG_INF, r2 = h2 ? Lb[1][c2p[k]] : KB_NEG_INF;
          const float t3 = lsp + sp + l1 + r2;
          const float t4 = lsp + sp + r1 + l2;
          const float m5 = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), t4);
          const float ms = fsafe(m5);
          const float s5 =
              exp2_hw(t0 - ms) + exp2_hw(t1 - ms) + exp2_hw(t2 - ms) + exp2_hw(t3 - ms) + exp2_hw(t4 - ms);
          lse_merge(m[k], acc[k], m5, s5);
        }
      }
    }
    __syncthreads();  // the staging buffers become the sweep buffers
#pragma unroll
    for (int k = 0; k < CPT; ++k) v[k] = log2_hw(acc[k]) + m[k];
    if (P.dts_out) {  // the backward reuses the split term at Pi*
      float* dst = P.dts_out + (size_t)row * S;
#pragma unroll
      for (int k = 0; k < CPT; ++k)
        if (own_pos_c<NT, CPT>(k) < S) dst[own_pos_c<NT, CPT>(k)] = v[k];
    }
  }
  if (tid < 64) {  // padding slots read by the child gathers (after the staging)
    X[MAXS + tid] = 0.0f;
    Q[MAXS + tid] = 0.0f;
  }

  // ---- linear space relative to the row maximum
  float lm = KB_NEG_INF;
#pragma unroll
  for (int k = 0; k < CPT; ++k) lm = fmaxf(lm, v[k]);
  const float Ms = fsafe(block_max1<NT>(lm, wM));
  const float leaf_lin = leaf_row ? exp2f(leaf_obs - Ms) : 0.0f;  // lpos = -1 for split rows
  float y[CPT], dl[CPT], cw[CPT], cwq[CPT];
  if constexpr (!EARLY) load_lin();
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = own_pos_c<NT, CPT>(k);
    const bool ok = i < S;
    y[k] = ok ? exp2f(v[k] - Ms) : 0.0f;
    dl[k] = leaf_row ? (i == lpos ? leaf_lin : 0.0f) : y[k];
    cw[k] = WEIGHTED ? (ok ? P.colw[i] : 0.0f) : 1.0f;
    cwq[k] = WEIGHTED ? (qp[k] < S ? P.colw[qp[k]] : 0.0f) : 1.0f;
  }
  int kexp = 0;
  float ps[CPT], rowsum = 0.0f, f = 1.0f;

  for (int sweep = 0;; ++sweep) {
    if constexpr (OMT) {  // (the launcher requires the tables for this shape)
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int c2 = ldg(fresh(P.om_tab + (size_t)OMT_C2 * MAXS + k * NT, sweep), tid);
        const int pn = ldg(fresh(P.om_tab + (size_t)OMT_PN * MAXS + k * NT, sweep), tid);
        c2p[k] = c2 >= 0 ? c2 : ZERO;
        qp[k] = pn & 0xffff;
        nex[k] = pn >> 16;
      }
    }
    // phase A: publish y; inclusive preorder scan (wavefront-local) in registers
    float sp[CPT], ta = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      ta += cw[k] * y[k];
      sp[k] = ta;
    }
    const float wa = wave_scan_incl(ta);
    lds_store_own<CPT>(X, y);
    if (lane == 63) wP[wv] = wa;
    __syncthreads();
    // phase B: preorder offsets and row sum; the postorder values and the
    // child2 values (read before the next barrier); exclusive postorder scan
    const float tp = lds_wave_values<NW>(wP, lane, 0.0f);
    float yq[CPT], x2[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      yq[k] = X[qp[k]];
      x2[k] = X[c2p[k]];
    }
    const float x1last = X[c1last];
    const float ip = wave_scan_first<NW>(tp);
    const float tsum = lane_value(ip, NW - 1);
    const float offp = lane_value(ip - tp, wv) + (wa - ta);
    float sq[CPT], tb = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      sq[k] = tb;
      tb += cwq[k] * yq[k];
    }
    const float wb = wave_scan_incl(tb);
    const float ob = wb - tb;
#pragma unroll
    for (int k = 0; k < CPT; ++k) sq[k] += ob;
    lds_store_own<CPT>(Q, sq);
    if (lane == 63) wQ[wv] = wb;
    const int e = tsum > 0.0f ? __builtin_amdgcn_frexp_expf(tsum) : 0;
    f = __builtin_amdgcn_ldexpf(1.0f, -e);
    kexp += e;
    rowsum = tsum * f;
    __syncthreads();
    // phase C: path sums ps(i) = Pre(i) - PostEx(tin(i) - i)
    const float tq = lds_wave_values<NW>(wQ, lane, 0.0f);
    const float iq = wave_scan_first<NW>(tq);
    const float eq = iq - tq;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int n = nex[k];
      ps[k] = (sp[k] + offp) - (Q[n] + __shfl(eq, n / SEG, 64));
    }
    if (sweep == P.n_sweeps) break;
    // y' = f (a y + k1 y[c1] + k2 y[c2] + emc (tsum - ps)) + dl 2^-kexp: f is a
    // power of two, so scaling the sum instead of each operand rounds the same
    const float scale = __builtin_amdgcn_ldexpf(1.0f, -kexp);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const float x1 = k + 1 < CPT ? y[k + 1] : x1last;
      float z = ca[k] * y[k];
      z += ck1[k] * x1;
      z += ck2[k] * x2[k];
      z += ce[k] * fmaxf(tsum - ps[k], 0.0f);
      y[k] = z * f + dl[k] * scale;
    }
  }

  // ---- outputs: Pi, Pibar from the final Pi, and the (weighted) row max
  const float M = Ms + (float)kexp;
  float piv[CPT], pbv[CPT];
  float lmax = KB_NEG_INF;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = own_pos_c<NT, CPT>(k);
    piv[k] = KB_NEG_INF;
    pbv[k] = KB_NEG_INF;
    if (i < S) {
      const float x = y[k] * f;
      piv[k] = x > 0.0f ? log2f(x) + M : KB_NEG_INF;
      const float na = rowsum - ps[k] * f;
      pbv[k] = na > 0.0f ? log2f(na) + M + P.mt[i] : KB_NEG_INF;
      lmax = fmaxf(lmax, WEIGHTED ? P.col[i] + piv[k] : piv[k]);
    }
  }
  // Lb[2], Lb[3] are unused since the staging
  lds_store_own<CPT>(Lb[2], piv);
  lds_store_own<CPT>(Lb[3], pbv);
  const float rmax = block_max1<NT>(lmax, wM);  // also publishes the staging
  const size_t rb = (size_t)row * S;
  float oa[CPT], ob[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sj = tid + j * NT;
    oa[j] = ob[j] = 0.0f;
    if (sj < S) {
      const int i = T.pre[sj];  // reloaded: keeps the table out of registers during the sweeps
      oa[j] = Lb[2][i];
      ob[j] = Lb[3][i];
      P.pi[rb + sj] = oa[j];
      P.pibar[rb + sj] = ob[j];
    }
  }
  if (tid == 0) P.rowmax[row] = rmax;
  // the rows identical to this one get the same outputs
  for (int d = P.dup_ptr[first + blockIdx.x]; d < P.dup_ptr[first + blockIdx.x + 1]; ++d) {
    const int r2 = P.dup_rows[d];
    const size_t b2 = (size_t)r2 * S;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int sj = tid + j * NT;
      if (sj < S) {
        P.pi[b2 + sj] = oa[j];
        P.pibar[b2 + sj] = ob[j];
      }
    }
    if (tid == 0) P.rowmax[r2] = rmax;
  }
}

#define KB_FWD_CASE(NT_, CPT_, KERNEL_)                                                                   \
  if (S <= NT_ * CPT_) {                                                                                  \
    if (P.use_col)                                                                                        \
      hipLaunchKernelGGL((KERNEL_<NT_, CPT_, true>), dim3(W), dim3(NT_), 0, st, P, first);                \
    else                                                                                                  \
      hipLaunchKernelGGL((KERNEL_<NT_, CPT_, false>), dim3(W), dim3(NT_), 0, st, P, first);               \
    return;                                                                                               \
  }


void launch_fwd_wave(const FwdParams& P, int first, int W, hipStream_t st) {
  if (W <= 0) return;
  const int S = P.S;
  if (P.wide == 1) {  // fewer, wider threads per row (tuning knob)
    KB_FWD_CASE(256, 8, fwd_row_kernel)
  }
  if (P.wide == 2 || (P.wide == 0 && W < P.narrow_below)) {  // more, narrower threads per row
    KB_FWD_CASE(1024, 2, fwd_row_kernel)
  }
  KB_FWD_CASE(64, 2, fwd_row_kernel)
  KB_FWD_CASE(128, 2, fwd_row_kernel)
  KB_FWD_CASE(256, 2, fwd_row_kernel)
  KB_FWD_CASE(256, 4, fwd_row_kernel)
  KB_FWD_CASE(512, 4, fwd_row_kernel)
  KB_FWD_CASE(1024, 4, fwd_row_kernel)
  if (P.om_tab && P.large) {
    KB_FWD_CASE(1024, 8, fwd_row_kernel)
  }
  KB_FWD_CASE(1024, 8, fwd_row_kernel_euler)
}

}  // namespace kb
