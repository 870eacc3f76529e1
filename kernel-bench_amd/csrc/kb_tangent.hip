// Forward tangents (JVP) of the solver's forward maps: the launchers beneath
// the drop-in replacements of the reference's kbench/core/kernels/
// e_step_tangent.py, dts_tangent.py and wave_tangent.py (declarations and
// the reference function each replaces: include/kbench_ops.h).
//
// Every map here is linear in the tangent at a frozen primal point, so each
// kernel splits into a primal set-up (softmax weights of the LSE terms, the
// linear row r = 2^(x - rowmax), the Pibar denominators), done once, and a
// tangent update that is an affine map of the tangent row:
//
//   dX_new[s] = K[s] + a[s] dX[s] + b[s] (dRS - dAS[s]) + c[s] dX[c1(s)] + d[s] dX[c2(s)]
//
// with dRS = sum_s r[s] dX[s] and dAS[s] = sum over the path root..s of
// r dX (one prefix scan over the Euler tour in LDS).  Fixed points and fixed
// iteration counts run inside one launch with the primal coefficients kept in
// registers and the tangent row in LDS, in float64 whatever the tensor dtype,
// except float32 rows too long for three float64 LDS rows (S > 6741), which
// run in float32.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>
#include <type_traits>

#include "kb_ops_common.hpp"

namespace kbo {

// ---- E-step tangent fixed point ------------------------------------------------------

template <typename T>
struct EtArgs {
  int G, S, use_col, max_iter;
  double tol;
  const T *E, *pS, *pD, *pL, *mt, *col, *dpS, *dpD, *dpL, *dmt, *dE0;
  T *dE, *dEs1, *dEs2, *dEbar;
  int* n_iter;
};

// One workgroup per item row g.  Primal at the frozen E*: r, denominators,
// the four E-step term weights w_k = 2^(t_k - E_new).  Tangent update:
//   dEbar = (dRS - dAS) / denom + dmt            (denom > 0, else 0)
//   dE_new = w0 (dpS + dE[c1] + dE[c2]) + w1 (dpD + 2 dE) + w2 (dE + dEbar) + w3 dpL
// (0 where E_new = -inf), iterated from dE0 (or 0) until
// max|dE_new - dE| <= tol * max(1, max|dE_new|) or max_iter steps.
template <typename T, int CPT, typename C = double>
__global__ __launch_bounds__(NT) void etan_kernel(OpsTree t, EtArgs<T> a) {
  extern __shared__ double smd[];  // raw storage: C values
  const int S = t.S;
  C* D = reinterpret_cast<C*>(smd);       // E row, then the tangent row
  C* EV = reinterpret_cast<C*>(smd) + S;  // 2S Euler scan
  __shared__ C red[NW];
  const C NI = ninf<C>();
  const size_t base = (size_t)blockIdx.x * S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) D[s] = (C)a.E[base + s];
  }
  __syncthreads();
  C r[CPT], K[CPT], w0[CPT], lin[CPT], wb[CPT], den[CPT], dm[CPT];
  bool pos[CPT];
  {
    C wE[CPT];
    C lm = NI;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      wE[k] = NI;
      if (s < S) {
        wE[k] = D[s] + (a.use_col ? (C)a.col[s] : C(0));
        lm = fmax(lm, wE[k]);
      }
    }
    const C M = block_max(lm, red);
    const C Ms = M == NI ? C(0) : M;
    C ls = C(0);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      r[k] = s < S ? xexp2(wE[k] - Ms) : C(0);
      ls += r[k];
    }
    const C rowsum = block_sum(ls, red);
    C anc[CPT];
    reg_path_sums<CPT>(t, r, anc, EV, red);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      K[k] = w0[k] = lin[k] = wb[k] = dm[k] = C(0);
      den[k] = C(1);
      pos[k] = false;
      if (s < S) {
        const size_t i = base + s;
        const C E = D[s];
        const int c1 = t.c1[s], c2 = t.c2[s];
        const C Es1 = c1 >= 0 ? D[c1] : NI, Es2 = c2 >= 0 ? D[c2] : NI;
        const C denom = rowsum - anc[k];
        pos[k] = denom > C(0);
        den[k] = pos[k] ? denom : C(1);
        const C Eb = pos[k] ? xlog2(den[k]) + M + (C)a.mt[i] : NI;
        const C t0 = (C)a.pS[i] + Es1 + Es2;
        const C t1 = (C)a.pD[i] + C(2) * E;
        const C t2 = E + Eb;
        const C t3 = (C)a.pL[i];
        const C m = fmax(fmax(t0, t1), fmax(t2, t3));
        const C ms = m == NI ? C(0) : m;
        const C e0 = xexp2(t0 - ms), e1 = xexp2(t1 - ms), e2 = xexp2(t2 - ms), e3 = xexp2(t3 - ms);
        const C total = e0 + e1 + e2 + e3;
        const C En = xlog2(total) + m;
        dm[k] = pos[k] ? (C)a.dmt[i] : C(0);
        if (En != NI && total > C(0)) {
          const C inv = C(1) / total;
          w0[k] = e0 * inv;
          const C w1 = e1 * inv, w2 = e2 * inv, w3 = e3 * inv;
          K[k] = w0[k] * (C)a.dpS[i] + w1 * (C)a.dpD[i] + w3 * (C)a.dpL[i] + w2 * dm[k];
          lin[k] = C(2) * w1 + w2;
          wb[k] = pos[k] ? w2 : C(0);
        }
      }
    }
    __syncthreads();  // every read of the E row is done
  }
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) D[s] = a.dE0 ? (C)a.dE0[base + s] : C(0);
  }
  __syncthreads();

  // q[k] = dRS - dAS[s]; reads D, leaves it untouched.
  auto tangent_q = [&](C (&q)[CPT]) {
    C x[CPT];
    C lsum = C(0);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      x[k] = s < S ? r[k] * D[s] : C(0);
      lsum += x[k];
    }
    const C dRS = block_sum(lsum, red);
    C dAS[CPT];
    reg_path_sums<CPT>(t, x, dAS, EV, red);
#pragma unroll
    for (int k = 0; k < CPT; ++k) q[k] = dRS - dAS[k];
  };

  // Float32 arithmetic cannot resolve a relative change below its own
  // rounding: its tolerance is floored at 8 float32 epsilons (9.5e-7), or a
  // tol below that would run every row to max_iter on 1-ulp oscillations.
  const C tol = std::is_same_v<C, float> ? (C)fmax(a.tol, 8.0 * (double)FLT_EPSILON) : (C)a.tol;
  int it = 0;
  for (;;) {
    C q[CPT], nx[CPT];
    tangent_q(q);
    C ld = C(0), lsc = C(0);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      nx[k] = C(0);
      if (s < S) {
        const int c1 = t.c1[s], c2 = t.c2[s];
        const C ch = (c1 >= 0 ? D[c1] : C(0)) + (c2 >= 0 ? D[c2] : C(0));
        nx[k] = K[k] + w0[k] * ch + lin[k] * D[s] + wb[k] * (q[k] / den[k]);
        ld = fmax(ld, fabs(nx[k] - D[s]));
        lsc = fmax(lsc, fabs(nx[k]));
      }
    }
    __syncthreads();  // every read of D is done
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) D[s] = nx[k];
    }
    ++it;
    const C md = block_max(ld, red);  // its barriers also publish D
    const C sc = block_max(lsc, red);
    if (md <= tol * fmax(C(1), sc) || it >= a.max_iter) break;
  }
  // children and Ebar tangents at the final dE
  C q[CPT];
  tangent_q(q);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      const size_t i = base + s;
      const int c1 = t.c1[s], c2 = t.c2[s];
      a.dE[i] = (T)D[s];
      a.dEs1[i] = (T)(c1 >= 0 ? D[c1] : C(0));
      a.dEs2[i] = (T)(c2 >= 0 ? D[c2] : C(0));
      a.dEbar[i] = (T)(pos[k] ? q[k] / den[k] + dm[k] : C(0));
    }
  }
  if (a.n_iter && threadIdx.x == 0) a.n_iter[blockIdx.x] = it;
}

// ---- split-term tangent ---------------------------------------------------------------

template <typename T>
struct DtArgs {
  int S, W, by_state;
  long long item_offset, prow;
  const T *Pi, *Pibar, *dPi, *dPibar, *lsp, *pD, *pS, *dpD, *dpS, *dts;
  const int64_t *sl, *sr, *item, *c1, *c2;
  const int *ptr, *order;
  T* out;
};

// One workgroup per wave row w: out[w, s] = sum over the row's splits (in
// increasing split order) of sum_k 2^(t_k - dts[w, s]) dt_k, 0 where
// dts[w, s] = -inf.
template <typename T, int CPT>
__global__ __launch_bounds__(NT) void dts_tan_kernel(DtArgs<T> a) {
  const int S = a.S;
  const int w = blockIdx.x;
  const T NI = ninf<T>();
  const int b = a.ptr[w], e = a.ptr[w + 1];
  const long long item = a.item[a.item_offset + w];
  const size_t pb = (size_t)(item * a.prow);
  double acc[CPT];
  T base[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    acc[k] = 0.0;
    base[k] = s < S ? a.dts[(size_t)w * S + s] : NI;
  }
  for (int j = b; j < e; ++j) {
    const int si = a.order[j];
    const size_t ol = (size_t)a.sl[si] * S, orr = (size_t)a.sr[si] * S;
    const T lsp = a.lsp[si];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S && base[k] != NI) {
        const T d = a.by_state ? a.pD[pb + s] : a.pD[pb];
        const T sp = a.by_state ? a.pS[pb + s] : a.pS[pb];
        const T dd = a.by_state ? a.dpD[pb + s] : a.dpD[pb];
        const T dsp = a.by_state ? a.dpS[pb + s] : a.dpS[pb];
        const int c1 = child_at(a.c1, s, S), c2 = child_at(a.c2, s, S);
        const T pl = a.Pi[ol + s], pr = a.Pi[orr + s];
        const T l1 = c1 >= 0 ? a.Pi[ol + c1] : NI, r1 = c1 >= 0 ? a.Pi[orr + c1] : NI;
        const T l2 = c2 >= 0 ? a.Pi[ol + c2] : NI, r2 = c2 >= 0 ? a.Pi[orr + c2] : NI;
        const T dpl = a.dPi[ol + s], dpr = a.dPi[orr + s];
        const T dl1 = c1 >= 0 ? a.dPi[ol + c1] : T(0), dr1 = c1 >= 0 ? a.dPi[orr + c1] : T(0);
        const T dl2 = c2 >= 0 ? a.dPi[ol + c2] : T(0), dr2 = c2 >= 0 ? a.dPi[orr + c2] : T(0);
        const T bs = base[k];
        const double v0 = (double)xexp2(lsp + d + pl + pr - bs) * (double)(dd + dpl + dpr);
        const double v1 = (double)xexp2(lsp + pl + a.Pibar[orr + s] - bs) * (double)(dpl + a.dPibar[orr + s]);
        const double v2 = (double)xexp2(lsp + pr + a.Pibar[ol + s] - bs) * (double)(dpr + a.dPibar[ol + s]);
        const double v3 = (double)xexp2(lsp + sp + l1 + r2 - bs) * (double)(dsp + dl1 + dr2);
        const double v4 = (double)xexp2(lsp + sp + r1 + l2 - bs) * (double)(dsp + dr1 + dl2);
        acc[k] += v0 + v1 + v2 + v3 + v4;
      }
    }
  }
  T* out = a.out + (size_t)w * S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) out[s] = base[k] != NI ? (T)acc[k] : T(0);
  }
}

// ---- wave-step tangent (one step, or the fixed-count self-loop) ---------------------------

template <typename T>
struct WtArgs {
  int S, W, use_col, use_leaf, n_iters;
  long long ws, pi_ws, cstride;
  const T *Pi, *dPi_in;
  T *dPi_out, *dPibar;
  const T *dts, *ddts;
  const T *mt, *dmt, *DL, *dDL, *Ebar, *dEbar, *E, *dE, *SL1, *dSL1, *SL2, *dSL2, *col;
  const int64_t *item, *leaf_state;
  const T *leaf_logp, *dleaf_logp;
};

// One workgroup per wave row w.  Primal at Pi row pi_ws + w: the weights
// w_k = 2^(t_k - Pi_new) of the six sweep terms (and the split term), r and
// the Pibar denominators.  n_iters tangent updates of the row:
//   dpibar = (dRS - dAS) / denom + dmt                     (denom > 0, else 0)
//   dPi_new = sum_k w_k dt_k,  dt = (dDL + dPi, dPi + dEbar, dpibar + dE,
//             dSL1 + dPi[c1], dSL2 + dPi[c2], dleaf at the leaf state, d_dts)
// (0 where Pi_new = -inf); the final row goes to dPi_out row ws + w and the
// dpibar of the last update to dPibar row ws + w.
template <typename T, int CPT>
__global__ __launch_bounds__(NT) void wave_tan_kernel(OpsTree t, WtArgs<T> a) {
  extern __shared__ double smd[];
  const int S = t.S;
  double* D = smd;       // Pi row, then the tangent row
  double* EV = smd + S;  // 2S Euler scan
  __shared__ double red[NW];
  const double NI = -__builtin_inf();
  const int w = blockIdx.x;
  const long long grow = a.ws + w;
  const long long item = a.item[grow];
  const size_t cb = (size_t)(item * a.cstride);
  const size_t lb = (size_t)item * S;
  const size_t ib = (size_t)(a.pi_ws + w) * S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) D[s] = (double)a.Pi[ib + s];
  }
  __syncthreads();
  double r[CPT], K[CPT], lin[CPT], wb[CPT], w3[CPT], w4[CPT], den[CPT], dm[CPT];
  bool pos[CPT];
  {
    double wv[CPT];
    double lm = NI;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      wv[k] = NI;
      if (s < S) {
        wv[k] = D[s] + (a.use_col ? (double)a.col[s] : 0.0);
        lm = fmax(lm, wv[k]);
      }
    }
    const double M = block_max(lm, red);
    const double Ms = M == NI ? 0.0 : M;
    double ls = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      r[k] = s < S ? exp2(wv[k] - Ms) : 0.0;
      ls += r[k];
    }
    const double rowsum = block_sum(ls, red);
    double anc[CPT];
    reg_path_sums<CPT>(t, r, anc, EV, red);
    const long long lstate = a.use_leaf ? a.leaf_state[grow] : -1;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      K[k] = lin[k] = wb[k] = w3[k] = w4[k] = dm[k] = 0.0;
      den[k] = 1.0;
      pos[k] = false;
      if (s < S) {
        const size_t ci = cb + s;
        const double pi = D[s];
        const int c1 = t.c1[s], c2 = t.c2[s];
        const double ps1 = c1 >= 0 ? D[c1] : NI, ps2 = c2 >= 0 ? D[c2] : NI;
        const double denom = rowsum - anc[k];
        pos[k] = denom > 0.0;
        den[k] = pos[k] ? denom : 1.0;
        const double pibar = pos[k] ? log2(den[k]) + M + (double)a.mt[ci] : NI;
        dm[k] = pos[k] ? (double)a.dmt[ci] : 0.0;
        const bool hit = lstate == s;
        const double t0 = (double)a.DL[ci] + pi;
        const double t1 = pi + (double)a.Ebar[ci];
        const double t2 = pibar + (double)a.E[ci];
        const double t3 = (double)a.SL1[ci] + ps1;
        const double t4 = (double)a.SL2[ci] + ps2;
        const double t5 = hit ? (double)a.leaf_logp[lb + s] : NI;
        double m = fmax(fmax(fmax(t0, t1), fmax(t2, t3)), fmax(t4, t5));
        double td = NI;
        if (a.dts) {
          td = (double)a.dts[(size_t)w * S + s];
          m = fmax(m, td);
        }
        const double ms = m == NI ? 0.0 : m;
        const double e0 = exp2(t0 - ms), e1 = exp2(t1 - ms), e2 = exp2(t2 - ms), e3 = exp2(t3 - ms);
        const double e4 = exp2(t4 - ms), e5 = exp2(t5 - ms), ed = a.dts ? exp2(td - ms) : 0.0;
        const double total = e0 + e1 + e2 + e3 + e4 + e5 + ed;
        const double res = log2(total) + m;
        if (res != NI && total > 0.0) {
          const double inv = 1.0 / total;
          double k0 = e0 * (double)a.dDL[ci] + e1 * (double)a.dEbar[ci] + e2 * ((double)a.dE[ci] + dm[k]) +
                      e3 * (double)a.dSL1[ci] + e4 * (double)a.dSL2[ci];
          if (hit) k0 += e5 * (double)a.dleaf_logp[lb + s];
          if (a.dts) k0 += ed * (double)a.ddts[(size_t)w * S + s];
          K[k] = k0 * inv;
          lin[k] = (e0 + e1) * inv;
          wb[k] = pos[k] ? e2 * inv : 0.0;
          w3[k] = e3 * inv;
          w4[k] = e4 * inv;
        }
      }
    }
    __syncthreads();  // every read of the Pi row is done
  }
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) D[s] = (double)a.dPi_in[ib + s];
  }
  __syncthreads();
  double dpb[CPT];
  const int n_it = a.n_iters < 1 ? 1 : a.n_iters;
  for (int it = 0; it < n_it; ++it) {
    double x[CPT];
    double lsum = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      x[k] = s < S ? r[k] * D[s] : 0.0;
      lsum += x[k];
    }
    const double dRS = block_sum(lsum, red);
    double dAS[CPT];
    reg_path_sums<CPT>(t, x, dAS, EV, red);
    double nx[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      nx[k] = 0.0;
      dpb[k] = 0.0;
      if (s < S) {
        const double qd = (dRS - dAS[k]) / den[k];
        dpb[k] = pos[k] ? qd + dm[k] : 0.0;
        const int c1 = t.c1[s], c2 = t.c2[s];
        nx[k] = K[k] + lin[k] * D[s] + wb[k] * qd + w3[k] * (c1 >= 0 ? D[c1] : 0.0) +
                w4[k] * (c2 >= 0 ? D[c2] : 0.0);
      }
    }
    __syncthreads();  // every read of D is done
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) D[s] = nx[k];
    }
    __syncthreads();
  }
  T* out = a.dPi_out + (size_t)grow * S;
  T* pb = a.dPibar ? a.dPibar + (size_t)grow * S : nullptr;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      out[s] = (T)D[s];
      if (pb) pb[s] = (T)dpb[k];
    }
  }
}

// float32 rows: the same update at preorder ownership (thread t owns
// positions t*CPT + k, as the forward row kernels), computed in float32 as the
// reference's Triton kernel computes it.  The path sums come from an
// inclusive preorder scan and an exclusive postorder scan,
//   dAS(i) = Pre(i) - PostEx(tin(i) - i),
// so one tangent update takes two barriers (the float64 kernel above takes an
// Euler-tour scan and two more barriers per update).
template <int CPT>
__global__ __launch_bounds__(NT) void wave_tan_pre_kernel(OpsTree t, WtArgs<float> a) {
  constexpr int MAXS = NT * CPT;
  constexpr int LD = MAXS + 64;
  constexpr int ZERO = MAXS;     // padding slot: 0 in X
  constexpr int SEG = 64 * CPT;  // postorder slots per wavefront
  extern __shared__ __align__(16) unsigned char smraw[];
  float* R = reinterpret_cast<float*>(smraw);  // the row at preorder positions: Pi, then the tangent
  float* X = R + LD;                           // the scanned values at preorder positions
  float* Q = X + LD;                           // exclusive postorder scan
  __shared__ float wM[NW], wA[NW], wB[NW];
  const int S = t.S;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const float NI = -__builtin_inff();
  const int w = blockIdx.x;
  const long long grow = a.ws + w;
  const long long item = a.item[grow];
  const size_t cb = (size_t)(item * a.cstride);
  const size_t lb = (size_t)item * S;
  const size_t ib = (size_t)(a.pi_ws + w) * S;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) R[t.ppos[sc]] = a.Pi[ib + sc];
  }
  if (tid < 64) X[MAXS + tid] = 0.0f;
  int c1p[CPT], c2p[CPT], nex[CPT], qp[CPT], colk[CPT];
  bool okp[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = kb::own_pos_c<NT, CPT>(k);
    okp[k] = i < S;
    c1p[k] = okp[k] ? t.pc1[i] : -1;
    c2p[k] = okp[k] ? t.pc2[i] : -1;
    nex[k] = okp[k] ? t.pnex[i] : 0;
    qp[k] = okp[k] ? t.ppost[i] : ZERO;
    colk[k] = okp[k] ? t.pcol[i] : 0;
  }
  __syncthreads();
  // ---- primal set-up at Pi: r = 2^(col + Pi - M), its row sum and path sums
  float pv[CPT], r[CPT];
  kb::lds_load_own<CPT>(R, pv);
  float lm = NI;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    if (!okp[k]) pv[k] = NI;
    lm = fmaxf(lm, (a.use_col && okp[k] ? a.col[colk[k]] : 0.0f) + pv[k]);
  }
  const float M = kb::block_max1<NT>(lm, wM);
  const float Ms = M == NI ? 0.0f : M;
  // one path-sum pass over x (own positions): tot = sum x, ps = Pre - PostEx;
  // x is published in X for the postorder reads.  Two barriers.
  float ps[CPT], tot = 0.0f;
  auto path_pass = [&](const float (&x)[CPT]) {
    float sp[CPT], ta = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      ta += x[k];
      sp[k] = ta;
    }
    const float wa = kb::wave_scan_incl(ta);
    kb::lds_store_own<CPT>(X, x);
    if (lane == 63) wA[wv] = wa;
    __syncthreads();
    const float tp = kb::lds_wave_values<NW>(wA, lane, 0.0f);
    float yq[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) yq[k] = X[qp[k]];
    const float ip = kb::wave_scan_first<NW>(tp);
    tot = kb::lane_value(ip, NW - 1);
    const float offp = kb::lane_value(ip - tp, wv) + (wa - ta);
    float sq[CPT], tb = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      sq[k] = tb;
      tb += yq[k];
    }
    const float wb = kb::wave_scan_incl(tb);
#pragma unroll
    for (int k = 0; k < CPT; ++k) sq[k] += wb - tb;
    kb::lds_store_own<CPT>(Q, sq);
    if (lane == 63) wB[wv] = wb;
    __syncthreads();
    const float tq = kb::lds_wave_values<NW>(wB, lane, 0.0f);
    const float eq = kb::wave_scan_first<NW>(tq) - tq;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int n = nex[k];
      ps[k] = (sp[k] + offp) - (Q[n] + __shfl(eq, n / SEG, 64));
    }
  };
#pragma unroll
  for (int k = 0; k < CPT; ++k)
    r[k] = okp[k] ? exp2f((a.use_col ? a.col[colk[k]] : 0.0f) + pv[k] - Ms) : 0.0f;
  path_pass(r);
  const float rowsum = tot;
  const long long lstate = a.use_leaf ? a.leaf_state[grow] : -1;
  float K[CPT], lin[CPT], wbk[CPT], w3[CPT], w4[CPT], den[CPT], dm[CPT];
  bool pos[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    K[k] = lin[k] = wbk[k] = w3[k] = w4[k] = dm[k] = 0.0f;
    den[k] = 1.0f;
    pos[k] = false;
    if (okp[k]) {
      const int s = colk[k];
      const size_t ci = cb + s;
      const float pi = pv[k];
      const float ps1 = c1p[k] >= 0 ? R[c1p[k]] : NI, ps2 = c2p[k] >= 0 ? R[c2p[k]] : NI;
      const float denom = rowsum - ps[k];
      pos[k] = denom > 0.0f;
      den[k] = pos[k] ? denom : 1.0f;
      const float pibar = pos[k] ? log2f(den[k]) + M + a.mt[ci] : NI;
      dm[k] = pos[k] ? a.dmt[ci] : 0.0f;
      const bool hit = lstate == s;
      const float t0 = a.DL[ci] + pi;
      const float t1 = pi + a.Ebar[ci];
      const float t2 = pibar + a.E[ci];
      const float t3 = a.SL1[ci] + ps1;
      const float t4 = a.SL2[ci] + ps2;
      const float t5 = hit ? a.leaf_logp[lb + s] : NI;
      float m = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), fmaxf(t4, t5));
      float td = NI;
      if (a.dts) {
        td = a.dts[(size_t)w * S + s];
        m = fmaxf(m, td);
      }
      const float ms = m == NI ? 0.0f : m;
      const float e0 = exp2f(t0 - ms), e1 = exp2f(t1 - ms), e2 = exp2f(t2 - ms), e3 = exp2f(t3 - ms);
      const float e4 = exp2f(t4 - ms), e5 = exp2f(t5 - ms), ed = a.dts ? exp2f(td - ms) : 0.0f;
      const float total = e0 + e1 + e2 + e3 + e4 + e5 + ed;
      const float res = log2f(total) + m;
      if (res != NI && total > 0.0f) {
        const float inv = 1.0f / total;
        float k0 = e0 * a.dDL[ci] + e1 * a.dEbar[ci] + e2 * (a.dE[ci] + dm[k]) + e3 * a.dSL1[ci] + e4 * a.dSL2[ci];
        if (hit) k0 += e5 * a.dleaf_logp[lb + s];
        if (a.dts) k0 += ed * a.ddts[(size_t)w * S + s];
        K[k] = k0 * inv;
        lin[k] = (e0 + e1) * inv;
        wbk[k] = pos[k] ? e2 * inv : 0.0f;
        w3[k] = e3 * inv;
        w4[k] = e4 * inv;
      }
    }
  }
  __syncthreads();  // every read of the Pi row in R is done
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) R[t.ppos[sc]] = a.dPi_in[ib + sc];
  }
  __syncthreads();
  float dv[CPT], dpb[CPT];
  kb::lds_load_own<CPT>(R, dv);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    if (!okp[k]) dv[k] = 0.0f;
    dpb[k] = 0.0f;
  }
  // ---- tangent updates.  The tangent row is published in R with the first
  // barrier of the pass (for the child reads, done before its second
  // barrier); the next update's writes follow that second barrier.
  const int n_it = a.n_iters < 1 ? 1 : a.n_iters;
  for (int it = 0; it < n_it; ++it) {
    if (it > 0) kb::lds_store_own<CPT>(R, dv);
    float x[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) x[k] = r[k] * dv[k];
    float ch1[CPT], ch2[CPT];
    {
      // (the pass's first barrier publishes R; the child reads precede its second)
      float sp[CPT], ta = 0.0f;
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        ta += x[k];
        sp[k] = ta;
      }
      const float wa = kb::wave_scan_incl(ta);
      kb::lds_store_own<CPT>(X, x);
      if (lane == 63) wA[wv] = wa;
      __syncthreads();
      const float tp = kb::lds_wave_values<NW>(wA, lane, 0.0f);
      float yq[CPT];
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        yq[k] = X[qp[k]];
        ch1[k] = c1p[k] >= 0 ? R[c1p[k]] : 0.0f;
        ch2[k] = c2p[k] >= 0 ? R[c2p[k]] : 0.0f;
      }
      const float ip = kb::wave_scan_first<NW>(tp);
      tot = kb::lane_value(ip, NW - 1);
      const float offp = kb::lane_value(ip - tp, wv) + (wa - ta);
      float sq[CPT], tb = 0.0f;
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        sq[k] = tb;
        tb += yq[k];
      }
      const float wb = kb::wave_scan_incl(tb);
#pragma unroll
      for (int k = 0; k < CPT; ++k) sq[k] += wb - tb;
      kb::lds_store_own<CPT>(Q, sq);
      if (lane == 63) wB[wv] = wb;
      __syncthreads();
      const float tq = kb::lds_wave_values<NW>(wB, lane, 0.0f);
      const float eq = kb::wave_scan_first<NW>(tq) - tq;
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int n = nex[k];
        ps[k] = (sp[k] + offp) - (Q[n] + __shfl(eq, n / SEG, 64));
      }
    }
    const float dRS = tot;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      float nx = 0.0f;
      dpb[k] = 0.0f;
      if (okp[k]) {
        const float qd = (dRS - ps[k]) / den[k];
        dpb[k] = pos[k] ? qd + dm[k] : 0.0f;
        nx = K[k] + lin[k] * dv[k] + wbk[k] * qd + w3[k] * ch1[k] + w4[k] * ch2[k];
      }
      dv[k] = nx;
    }
  }
  // outputs by column (coalesced): R and X were last read before the last
  // pass's second barrier
  kb::lds_store_own<CPT>(R, dv);
  kb::lds_store_own<CPT>(X, dpb);
  __syncthreads();
  float* out = a.dPi_out + (size_t)grow * S;
  float* pb = a.dPibar ? a.dPibar + (size_t)grow * S : nullptr;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) {
      const int i = t.ppos[sc];
      out[sc] = R[i];
      if (pb) pb[sc] = X[i];
    }
  }
}

}  // namespace kbo

using namespace kbo_host;

namespace {

template <typename T, int CPT>
int launch_etan(const kbo::OpsTree& t, const kbo::EtArgs<T>& a, bool f32, size_t lds, hipStream_t st) {
  if constexpr (std::is_same_v<T, float> && CPT == 8) {
    if (f32) {  // rows too long for three float64 LDS rows
      auto k = kbo::etan_kernel<T, CPT, float>;
      if (int rc = set_lds(k, lds)) return rc;
      hipLaunchKernelGGL(k, dim3(a.G), dim3(kbo::NT), lds, st, t, a);
      return 0;
    }
  }
  if (f32) return kb::set_error(KB_ERR_ARG, "S=%d: no float32 etan_kernel for %d positions per thread", a.S, CPT);
  auto k = kbo::etan_kernel<T, CPT>;
  if (int rc = set_lds(k, lds)) return rc;
  hipLaunchKernelGGL(k, dim3(a.G), dim3(kbo::NT), lds, st, t, a);
  return 0;
}

// float32 rows run the preorder-ownership kernel, float64 rows the float64 one
template <typename T, int CPT>
int launch_wave_tan(const kbo::OpsTree& t, const kbo::WtArgs<T>& a, int W, size_t lds, hipStream_t st) {
  if constexpr (std::is_same_v<T, float>) {
    const size_t lds_pre = (size_t)3 * (kbo::NT * CPT + 64) * sizeof(float);
    auto k = kbo::wave_tan_pre_kernel<CPT>;
    if (int rc = set_lds(k, lds_pre)) return rc;
    hipLaunchKernelGGL(k, dim3(W), dim3(kbo::NT), lds_pre, st, t, a);
    return 0;
  }
  // the float64 kernel keeps three float64 rows of S in LDS
  if (int rc = check_lds(lds, a.S, KB_F64)) return rc;
  auto k = kbo::wave_tan_kernel<T, CPT>;
  if (int rc = set_lds(k, lds)) return rc;
  hipLaunchKernelGGL(k, dim3(W), dim3(kbo::NT), lds, st, t, a);
  return 0;
}

}  // namespace

extern "C" {

int kb_e_tangent_fixed_point(const kb_tree* tr, const kb_etan_io* io, void* stream) {
  if (!tr || !io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->G < 0) return kb::set_error(KB_ERR_ARG, "G must be non-negative");
  if (io->max_iter < 1 || !(io->tol >= 0.0)) return kb::set_error(KB_ERR_ARG, "max_iter must be >= 1 and tol >= 0");
  if (io->G == 0) return 0;
  const int S = tr->S;
  size_t lds;
  bool f32;
  if (int rc = three_row_lds(S, io->dtype, &lds, &f32)) return rc;
  const kbo::OpsTree t = tr->dev();
  KBO_DISPATCH(io->dtype, S, {
    kbo::EtArgs<T> a{io->G, S, io->use_col_weights, io->max_iter, io->tol,
                     (const T*)io->E, (const T*)io->log_pS, (const T*)io->log_pD, (const T*)io->log_pL,
                     (const T*)io->max_coupling, (const T*)io->col_log_probs, (const T*)io->dlog_pS,
                     (const T*)io->dlog_pD, (const T*)io->dlog_pL, (const T*)io->dmax_coupling, (const T*)io->dE0,
                     (T*)io->dE, (T*)io->dE_s1, (T*)io->dE_s2, (T*)io->dEbar, io->n_iter};
    if (int rc = launch_etan<T, CPT>(t, a, f32, lds, st_of(stream))) return rc;
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_dts_tangent(const kb_dts_tan_io* io, void* stream) {
  if (!io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->W < 0 || io->N < 0 || io->S < 1) return kb::set_error(KB_ERR_ARG, "bad sizes W=%d N=%lld S=%d", io->W,
                                                                (long long)io->N, io->S);
  if (io->W == 0) return 0;
  const int S = io->S;
  KBO_DISPATCH(io->dtype, S, {
    kbo::DtArgs<T> a{S, io->W, io->param_by_state, io->item_offset, io->param_row_stride,
                     (const T*)io->Pi, (const T*)io->Pibar, (const T*)io->dPi, (const T*)io->dPibar,
                     (const T*)io->log_split_probs, (const T*)io->log_pD, (const T*)io->log_pS,
                     (const T*)io->dlog_pD, (const T*)io->dlog_pS, (const T*)io->dts_r,
                     io->sl, io->sr, io->item_idx, io->node_child1, io->node_child2,
                     io->split_ptr, io->split_order, (T*)io->out};
    hipLaunchKernelGGL((kbo::dts_tan_kernel<T, CPT>), dim3(io->W), dim3(kbo::NT), 0, st_of(stream), a);
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_wave_step_tangent(const kb_tree* tr, const kb_wave_tan_io* io, void* stream) {
  if (!tr || !io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->S != tr->S) return kb::set_error(KB_ERR_ARG, "S=%d does not match the tree (%d)", io->S, tr->S);
  if (io->W < 0) return kb::set_error(KB_ERR_ARG, "W must be non-negative");
  if ((io->dts == nullptr) != (io->d_dts == nullptr))
    return kb::set_error(KB_ERR_ARG, "dts and d_dts must be given together");
  if (io->W == 0) return 0;
  const int S = tr->S;
  const size_t lds = (size_t)3 * S * sizeof(double);
  const kbo::OpsTree t = tr->dev();
  KBO_DISPATCH(io->dtype, S, {
    kbo::WtArgs<T> a{S, io->W, io->use_col_weights, io->use_leaf_index, io->n_iters, io->ws, io->pi_ws,
                     io->const_stride, (const T*)io->Pi_in, (const T*)io->dPi_in, (T*)io->dPi_out,
                     (T*)io->dPibar_out, (const T*)io->dts, (const T*)io->d_dts,
                     (const T*)io->max_coupling, (const T*)io->dMC, (const T*)io->DL, (const T*)io->dDL,
                     (const T*)io->Ebar, (const T*)io->dEbar, (const T*)io->E, (const T*)io->dE,
                     (const T*)io->SL1, (const T*)io->dSL1, (const T*)io->SL2, (const T*)io->dSL2,
                     (const T*)io->col_log_probs, io->item_idx, io->leaf_state, (const T*)io->leaf_logp,
                     (const T*)io->dleaf_logp};
    if (int rc = launch_wave_tan<T, CPT>(t, a, io->W, lds, st_of(stream))) return rc;
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
