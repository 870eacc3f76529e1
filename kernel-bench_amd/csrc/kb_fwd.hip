// Fused forward wave kernel: one workgroup per clade row does the split
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
// The sweeps run in linear space: x = 2^(Pi - M) with a per-row exponent M that
// is renormalised by an exact power of two after every sweep, so a sweep is
//   y = a x + emc NA(x) + k1 x[c1] + k2 x[c2] + (leaf | dts) 2^-M
// with per-column constants a = 2^DL + 2^Ebar, emc = 2^(E+mt), k1 = 2^SL1,
// k2 = 2^SL2 prepared once per solve.
#include "kb_device.hpp"
#include "kb_kernels.hpp"

namespace kb {

template <int NT, int CPT>
__global__ __launch_bounds__(NT) void fwd_wave_kernel(FwdParams P, int first) {
  constexpr int MAXS = NT * CPT;
  __shared__ float X[MAXS];
  __shared__ float B0[MAXS];
  __shared__ float B1[MAXS];
  __shared__ float red[NT / 64];

  const int S = P.S;
  const int tid = threadIdx.x;
  const int row = P.sched_rows[first + blockIdx.x];
  const int leaf_wave = P.row_kind[row];
  const int item = P.item[row];
  const size_t cb = (size_t)item * P.const_stride;

  float v[CPT];
  int leaf = -1;
  float leaf_obs = 0.0f;
  if (leaf_wave) {
    leaf = P.leaf_state[row];
    const int ls = P.tr.sub_start[leaf], le = P.tr.sub_end[leaf];
    leaf_obs = P.leaf_logp[cb + leaf];
    const float leaf_col = P.use_col ? P.col[leaf] : 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      v[k] = KB_NEG_INF;
      if (s < S) {
        const bool hit = s == leaf;
        const int st = P.tr.sub_start[s];
        const bool desc = st >= ls && st < le;
        const float pi_w = hit ? leaf_obs : KB_NEG_INF;
        const float pibar_w = desc ? KB_NEG_INF : P.mt[cb + s] + leaf_col + leaf_obs;
        const float pi_s1 = P.tr.c1[s] == leaf ? leaf_obs : KB_NEG_INF;
        const float pi_s2 = P.tr.c2[s] == leaf ? leaf_obs : KB_NEG_INF;
        const float t0 = P.DL[cb + s] + pi_w;
        const float t1 = pi_w + P.Ebar[cb + s];
        const float t2 = pibar_w + P.E[cb + s];
        const float t3 = P.SL1[cb + s] + pi_s1;
        const float t4 = P.SL2[cb + s] + pi_s2;
        const float t5 = hit ? P.leaf_logp[cb + s] : KB_NEG_INF;
        float m = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), fmaxf(t4, t5));
        float ms = fsafe(m);
        float sum = exp2f(t0 - ms) + exp2f(t1 - ms) + exp2f(t2 - ms) + exp2f(t3 - ms) + exp2f(t4 - ms) +
                    exp2f(t5 - ms);
        v[k] = log2f(sum) + m;
      }
    }
  } else {
    float m[CPT], acc[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      m[k] = KB_NEG_INF;
      acc[k] = 0.0f;
    }
    const int b = P.split_ptr[row], e = P.split_ptr[row + 1];
    for (int i = b; i < e; ++i) {
      const size_t l = (size_t)P.split_l[i] * S, r = (size_t)P.split_r[i] * S;
      const float lsp = P.split_lsp[i];
      const float* Pl = P.pi + l;
      const float* Pr = P.pi + r;
      const float* Bl = P.pibar + l;
      const float* Br = P.pibar + r;
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int s = tid + k * NT;
        if (s < S) {
          const int a1 = P.tr.c1[s], a2 = P.tr.c2[s];
          const float pl = Pl[s], pr = Pr[s];
          const float d = P.pD.at(item, s), sp = P.pS.at(item, s);
          const float t0 = lsp + d + pl + pr;
          const float t1 = lsp + pl + Br[s];
          const float t2 = lsp + pr + Bl[s];
          const float l1 = a1 >= 0 ? Pl[a1] : KB_NEG_INF, r1 = a1 >= 0 ? Pr[a1] : KB_NEG_INF;
          const float l2 = a2 >= 0 ? Pl[a2] : KB_NEG_INF, r2 = a2 >= 0 ? Pr[a2] : KB_NEG_INF;
          const float t3 = lsp + sp + l1 + r2;
          const float t4 = lsp + sp + r1 + l2;
          float m5 = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), t4);
          float ms = fsafe(m5);
          float s5 = exp2f(t0 - ms) + exp2f(t1 - ms) + exp2f(t2 - ms) + exp2f(t3 - ms) + exp2f(t4 - ms);
          lse_merge(m[k], acc[k], m5, s5);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k) v[k] = log2f(acc[k]) + m[k];
  }

  // ---- to linear space with an exact power-of-two row scale
  float lm = KB_NEG_INF;
#pragma unroll
  for (int k = 0; k < CPT; ++k)
    if (tid + k * NT < S) lm = fmaxf(lm, v[k]);
  const float M0 = block_max<NT>(lm, red);
  const float Ms = fsafe(M0);
  float x[CPT], dl[CPT], ca[CPT], ce[CPT], ck1[CPT], ck2[CPT], cw[CPT];
  int c1[CPT], c2[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = tid + k * NT;
    const bool ok = s < S;
    x[k] = ok ? exp2f(v[k] - Ms) : 0.0f;
    dl[k] = leaf_wave ? 0.0f : x[k];
    ca[k] = ok ? P.lin_a[cb + s] : 0.0f;
    ce[k] = ok ? P.lin_emc[cb + s] : 0.0f;
    ck1[k] = ok ? P.lin_k1[cb + s] : 0.0f;
    ck2[k] = ok ? P.lin_k2[cb + s] : 0.0f;
    cw[k] = ok ? (P.use_col ? P.colw[s] : 1.0f) : 0.0f;
    c1[k] = ok ? P.tr.c1[s] : -1;
    c2[k] = ok ? P.tr.c2[s] : -1;
  }
  const float leaf_lin = leaf_wave ? exp2f(P.leaf_logp[cb + leaf] - Ms) : 0.0f;
  int kexp = 0;

  for (int sweep = 0; sweep < P.n_sweeps; ++sweep) {
    float ls = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      if (s < S) {
        X[s] = x[k];
        B0[s] = cw[k] * x[k];
        ls += cw[k] * x[k];
      }
    }
    const float rowsum = block_sum<NT>(ls, red);
    const float* ps = path_sum_lds<NT, CPT>(P.tr, B0, B1);
    const float scale = ldexpf(1.0f, -kexp);
    float y[CPT];
    float ymax = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      float yy = 0.0f;
      if (s < S) {
        float na = rowsum - ps[s];
        na = na > 0.0f ? na : 0.0f;
        yy = ca[k] * x[k] + ce[k] * na;
        if (c1[k] >= 0) yy += ck1[k] * X[c1[k]];
        if (c2[k] >= 0) yy += ck2[k] * X[c2[k]];
        if (leaf_wave) {
          if (s == leaf) yy += leaf_lin * scale;
        } else {
          yy += dl[k] * scale;
        }
      }
      y[k] = yy;
      ymax = fmaxf(ymax, yy);
    }
    const float gmax = block_max<NT>(ymax, red);  // barrier: LDS reads above are complete
    if (gmax > 0.0f) {
      int e;
      frexpf(gmax, &e);
#pragma unroll
      for (int k = 0; k < CPT; ++k) x[k] = ldexpf(y[k], -e);
      kexp += e;
    } else {
#pragma unroll
      for (int k = 0; k < CPT; ++k) x[k] = y[k];
    }
  }

  // ---- outputs: Pi, Pibar from the final Pi, and the (weighted) row max
  const float M = Ms + (float)kexp;
  const size_t rb = (size_t)row * S;
  float ls = 0.0f, lmax = KB_NEG_INF;
  float piv[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = tid + k * NT;
    if (s < S) {
      piv[k] = x[k] > 0.0f ? log2f(x[k]) + M : KB_NEG_INF;
      P.pi[rb + s] = piv[k];
      lmax = fmaxf(lmax, P.use_col ? P.col[s] + piv[k] : piv[k]);
      B0[s] = cw[k] * x[k];
      ls += cw[k] * x[k];
    }
  }
  const float rowsum = block_sum<NT>(ls, red);
  const float* ps = path_sum_lds<NT, CPT>(P.tr, B0, B1);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = tid + k * NT;
    if (s < S) {
      float na = rowsum - ps[s];
      P.pibar[rb + s] = na > 0.0f ? log2f(na) + M + P.mt[cb + s] : KB_NEG_INF;
    }
  }
  const float rmax = block_max<NT>(lmax, red);
  if (tid == 0) P.rowmax[row] = rmax;
}

#define KB_FWD_CASE(NT_, CPT_)                                                                   \
  if (S <= NT_ * CPT_) {                                                                         \
    hipLaunchKernelGGL((fwd_wave_kernel<NT_, CPT_>), dim3(W), dim3(NT_), 0, st, P, first);        \
    return;                                                                                      \
  }

void launch_fwd_wave(const FwdParams& P, int first, int W, hipStream_t st) {
  if (W <= 0) return;
  const int S = P.S;
  KB_FWD_CASE(64, 1)
  KB_FWD_CASE(128, 1)
  KB_FWD_CASE(256, 1)
  KB_FWD_CASE(256, 2)
  KB_FWD_CASE(512, 2)
  KB_FWD_CASE(512, 4)
  KB_FWD_CASE(1024, 4)
  KB_FWD_CASE(1024, 8)
}

}  // namespace kb
