// Parameter extraction, E-step fixed point, forward constants and the loss.
//
// Everything here is O(S) work (one species-tree-sized vector), so it runs in
// a single workgroup and in float64: the reference's stopping rule
// max|E_new - E| < e_tol (pristine e_step.py:482-493, e_tol = 1e-8) sits below
// float32 resolution for |E| >= 0.125, so a float32 iterate can cycle at the
// last bit until e_max_iter.  In float64 the same rule is reached, and the
// outputs are rounded to float32 once.
//
// The E-step map is evaluated in linear space: with e = 2^E,
//   e_new = 2^pS e[c1] e[c2] + 2^pD e^2 + e * 2^mt * NA(e) + 2^pL,
//   NA(e)[s] = sum over j not an ancestor-or-self of s of (w_j e_j),
// which is the reference's log-space update (pristine e_step.py:42-91) written
// without transcendentals.  NA = rowsum - pathsum as in the reference.
#include "kb_device.hpp"
#include "kb_kernels.hpp"

namespace kb {

// Top-down path sums in place over all nodes grouped by depth (root first).
template <int NT>
__device__ __forceinline__ void path_sum_levels_inplace(const EStepParams& P, double* v) {
  for (int d = 1; d < P.n_tlevels; ++d) {
    const int b = P.tlevel_ptr[d], e = P.tlevel_ptr[d + 1];
    for (int i = b + threadIdx.x; i < e; i += NT) {
      int n = P.tlevel_node[i];
      v[n] += v[P.tr.parent[n]];
    }
    __syncthreads();
  }
}

constexpr int ENT = 1024;

// Path sums in place: one Euler-tour scan when its scratch fits in LDS, else by levels.
template <int EMAXS>
__device__ __forceinline__ void path_sums(const EStepParams& P, double* v, double* scan2, double* red) {
  if constexpr (EMAXS <= 4096)
    euler_path_sums_f64<ENT>(P.ts, v, scan2, red);
  else
    path_sum_levels_inplace<ENT>(P, v);
}

template <int EMAXS>
__global__ __launch_bounds__(ENT) void estep_fixed_point_kernel(EStepParams P) {
  constexpr int ECPT = EMAXS / ENT;
  __shared__ double ev[EMAXS];
  __shared__ double pv[EMAXS];
  __shared__ double scan2[EMAXS <= 4096 ? 2 * EMAXS : 1];  // Euler-tour scan (small trees)
  __shared__ double red[ENT / 64];
  __shared__ int ired[ENT / 64];
  const int S = P.S;
  const int tid = threadIdx.x;
  const double LN2 = 0.6931471805599453;

  double pS[ECPT], pD[ECPT], pL[ECPT], pT[ECPT], mt[ECPT], cl[ECPT], w[ECPT], e[ECPT];
  int c1[ECPT], c2[ECPT];

  // ---- parameters: log2-softmax of [0, theta] (extract_parameters.py:25-34)
#pragma unroll
  for (int k = 0; k < ECPT; ++k) {
    int s = tid + k * ENT;
    pS[k] = pD[k] = pL[k] = pT[k] = 0.0;
    c1[k] = c2[k] = -1;
    if (s < S) {
      const float* th = P.statewise ? P.theta + 3 * (size_t)s : P.theta;
      double l0 = 0.0, l1 = th[0], l2 = th[1], l3 = th[2];
      double mx = fmax(fmax(l0, l1), fmax(l2, l3));
      double lse = mx + log2(exp2(l0 - mx) + exp2(l1 - mx) + exp2(l2 - mx) + exp2(l3 - mx));
      pS[k] = l0 - lse;
      pD[k] = l1 - lse;
      pL[k] = l2 - lse;
      pT[k] = l3 - lse;
      c1[k] = P.tr.c1[s];
      c2[k] = P.tr.c2[s];
    }
  }

  // ---- column log-probabilities and max_coupling
  if (P.use_col) {
    // col_log_probs = log_softmax(col_weights) / ln2 (extract_parameters.py:37-38)
    double lmax = -__builtin_inf();
#pragma unroll
    for (int k = 0; k < ECPT; ++k) {
      int s = tid + k * ENT;
      if (s < S) lmax = fmax(lmax, (double)P.col_weights[s]);
    }
    double gmax = block_max<ENT>(lmax, red);
    double lsum = 0.0;
#pragma unroll
    for (int k = 0; k < ECPT; ++k) {
      int s = tid + k * ENT;
      if (s < S) lsum += exp((double)P.col_weights[s] - gmax);
    }
    double gsum = block_sum<ENT>(lsum, red);
    double lz = gmax + log(gsum);
#pragma unroll
    for (int k = 0; k < ECPT; ++k) {
      int s = tid + k * ENT;
      if (s < S) {
        cl[k] = ((double)P.col_weights[s] - lz) / LN2;
        pv[s] = exp2(cl[k]);
      }
    }
    __syncthreads();
    path_sums<EMAXS>(P, pv, scan2, red);
    // col_valid_log_normalizer (extract_parameters.py:41-65), then mt = pT + norm
#pragma unroll
    for (int k = 0; k < ECPT; ++k) {
      int s = tid + k * ENT;
      if (s < S) {
        double valid = 1.0 - pv[s];
        double cn = valid > 0.0 ? -log2(fmax(valid, 2.2250738585072014e-308)) : -__builtin_inf();
        mt[k] = pT[k] + cn;
        w[k] = exp2(cl[k]);
      }
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int k = 0; k < ECPT; ++k) {
      int s = tid + k * ENT;
      if (s < S) {
        cl[k] = -log2((double)S);
        mt[k] = pT[k] + (double)P.unnorm_row_max[s];
        w[k] = 1.0;
      }
    }
  }

  // ---- E fixed point (pristine e_step.py:438-501) in linear float64
  double lin_pS[ECPT], lin_pD[ECPT], lin_pL[ECPT], lin_mt[ECPT];
#pragma unroll
  for (int k = 0; k < ECPT; ++k) {
    lin_pS[k] = exp2(pS[k]);
    lin_pD[k] = exp2(pD[k]);
    lin_pL[k] = exp2(pL[k]);
    lin_mt[k] = exp2(mt[k]);
    e[k] = exp2(P.e_init);
  }
  const double ratio_hi = exp2(P.tol), ratio_lo = exp2(-P.tol);
  int it = 0;
  for (;;) {
#pragma unroll
    for (int k = 0; k < ECPT; ++k) {
      int s = tid + k * ENT;
      if (s < S) {
        ev[s] = e[k];
        pv[s] = w[k] * e[k];
      }
    }
    double ls = 0.0;
#pragma unroll
    for (int k = 0; k < ECPT; ++k)
      if (tid + k * ENT < S) ls += w[k] * e[k];
    double rowsum = block_sum<ENT>(ls, red);  // also publishes ev/pv
    path_sums<EMAXS>(P, pv, scan2, red);
    int ok = 1;
#pragma unroll
    for (int k = 0; k < ECPT; ++k) {
      int s = tid + k * ENT;
      if (s < S) {
        double e1 = c1[k] >= 0 ? ev[c1[k]] : 0.0;
        double e2 = c2[k] >= 0 ? ev[c2[k]] : 0.0;
        double na = rowsum - pv[s];
        double eb = na > 0.0 ? lin_mt[k] * na : 0.0;
        double en = lin_pS[k] * e1 * e2 + lin_pD[k] * e[k] * e[k] + e[k] * eb + lin_pL[k];
        // |log2(en / e)| < tol without a log: en / e inside (2^-tol, 2^tol)
        const double ratio = en / e[k];
        if (!(ratio < ratio_hi && ratio > ratio_lo)) ok = 0;
        e[k] = en;
      }
    }
    ++it;
    // one barrier pair: every read of ev/pv above precedes the next overwrite
    int lok = ok;
    for (int o = 32; o > 0; o >>= 1) lok &= __shfl_xor(lok, o, 64);
    if ((tid & 63) == 0) ired[tid >> 6] = lok;
    __syncthreads();
    int all_ok = 1;
#pragma unroll
    for (int i = 0; i < ENT / 64; ++i) all_ok &= ired[i];
    __syncthreads();
    if (all_ok || it >= P.max_iter) break;
  }
  if (tid == 0 && P.n_iter_out) P.n_iter_out[0] = it;

  // ---- outputs from the final E (pristine e_step.py:495-499)
  double Ed[ECPT];
#pragma unroll
  for (int k = 0; k < ECPT; ++k) {
    int s = tid + k * ENT;
    Ed[k] = log2(e[k]);
    if (s < S) {
      ev[s] = Ed[k];
      pv[s] = w[k] * e[k];
    }
  }
  double ls = 0.0;
#pragma unroll
  for (int k = 0; k < ECPT; ++k)
    if (tid + k * ENT < S) ls += w[k] * e[k];
  double rowsum = block_sum<ENT>(ls, red);
  path_sums<EMAXS>(P, pv, scan2, red);
  const double NINF = -__builtin_inf();
#pragma unroll
  for (int k = 0; k < ECPT; ++k) {
    int s = tid + k * ENT;
    if (s < S) {
      double Es1 = c1[k] >= 0 ? ev[c1[k]] : NINF;
      double Es2 = c2[k] >= 0 ? ev[c2[k]] : NINF;
      double na = rowsum - pv[s];
      double Ebar = na > 0.0 ? log2(na) + mt[k] : NINF;
      double E = Ed[k];
      P.E[s] = (float)E;
      P.E_s1[s] = (float)Es1;
      P.E_s2[s] = (float)Es2;
      P.Ebar[s] = (float)Ebar;
      if (P.E64) P.E64[s] = E;
      P.mt[s] = (float)mt[k];
      P.col_log_probs[s] = (float)cl[k];
      if (P.statewise) {
        P.log_pS[s] = (float)pS[k];
        P.log_pD[s] = (float)pD[k];
        P.log_pL[s] = (float)pL[k];
      } else if (s == 0) {
        P.log_pS[0] = (float)pS[k];
        P.log_pD[0] = (float)pD[k];
        P.log_pL[0] = (float)pL[k];
      }
      // row-kernel constants at preorder positions
      const int i = P.pre[s];
      P.c_DL[i] = (float)(1.0 + pD[k] + E);
      P.c_SL1[i] = (float)(pS[k] + Es2);
      P.c_SL2[i] = (float)(pS[k] + Es1);
      P.c_pS[i] = (float)pS[k];
      P.c_pD[i] = (float)pD[k];
      P.c_colw[i] = (float)w[k];
      P.c_Ebar[i] = (float)Ebar;
      P.c_E[i] = (float)E;
      P.c_mt[i] = (float)mt[k];
      P.c_col[i] = (float)cl[k];
      P.lin_a[i] = (float)(exp2(1.0 + pD[k] + E) + exp2(Ebar));
      P.lin_emc[i] = (float)exp2(E + mt[k]);
      P.lin_k1[i] = (float)exp2(pS[k] + Es2);
      P.lin_k2[i] = (float)exp2(pS[k] + Es1);
    }
  }
}

// ---- E-step for trees of up to NT*CPT nodes: register-resident, preorder
// ownership (thread t owns positions t*CPT + k), two barriers per iteration.
// The path sum of w e at position i is Pre(i) - PostEx(tin(i) - i): the
// inclusive preorder prefix sum minus the exclusive postorder prefix sum (the
// nodes left before entering i are the first tin(i) - i nodes in postorder).
// Both scans run in registers (DPP); LDS holds e and w e for the child and
// postorder gathers and the wavefront-local postorder scan.  The convergence
// flags of an update are published with the next iteration's first barrier,
// whose path sums are then also the outputs' (same rule as the kernel above).

template <int NT, int CPT>
__global__ __launch_bounds__(NT) void estep_pre_kernel(EStepParams P) {
  constexpr int MAXS = NT * CPT;
  constexpr int NW = NT / 64;
  constexpr int ZERO = MAXS;     // padding slot: 0 in every buffer
  constexpr int SEG = 64 * CPT;  // postorder slots per wavefront
  __shared__ __align__(16) double Eb[MAXS + 64];  // e at positions (child gathers)
  __shared__ __align__(16) double Xw[MAXS + 64];  // w e at positions (postorder gathers)
  __shared__ __align__(16) double Qb[MAXS + 64];  // wavefront-local exclusive postorder scans
  __shared__ double wP[NW], wQ[NW], red[NW];
  __shared__ int wok[NW];
  const PreDev& T = P.pd;
  const int S = P.S;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const double LN2 = 0.6931471805599453;
  const double NINF = -__builtin_inf();

  int colk[CPT], c2p[CPT], nex[CPT], qp[CPT];
  bool h1[CPT], okp[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = tid * CPT + k;
    okp[k] = i < S;
    colk[k] = okp[k] ? T.col[i] : 0;
    const int a = okp[k] ? T.c1pos[i] : -1, b = okp[k] ? T.c2pos[i] : -1;
    h1[k] = a >= 0;  // child1 of i is i + 1 (preorder, child1 first)
    c2p[k] = b >= 0 ? b : ZERO;
    nex[k] = okp[k] ? T.tin[i] - i : 0;
    qp[k] = okp[k] ? T.post[i] : ZERO;
  }
  const int c1last = h1[CPT - 1] ? tid * CPT + CPT : ZERO;
  if (tid < 64) {
    Eb[MAXS + tid] = 0.0;
    Xw[MAXS + tid] = 0.0;
    Qb[MAXS + tid] = 0.0;
  }

  // ancestors-or-self sums of x at the own positions and the total; two
  // barriers (the padding writes above are published by the first)
  auto path_sums = [&](const double (&x)[CPT], double (&ps)[CPT], double& total) {
    double sp[CPT], ta = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      ta += x[k];
      sp[k] = ta;
    }
    const double wa = wave_scan_incl_f64(ta);
    lds_store_own_f64<CPT>(Xw, x);
    if (lane == 63) wP[wv] = wa;
    __syncthreads();
    const double tp = lds_wave_values<NW>(wP, lane, 0.0);
    double yq[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) yq[k] = Xw[qp[k]];
    const double ip = wave_scan_first_f64<NW>(tp);
    total = lane_value_f64(ip, NW - 1);
    const double offp = lane_value_f64(ip - tp, wv) + (wa - ta);
    double sq[CPT], tb = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      sq[k] = tb;
      tb += yq[k];
    }
    const double wb = wave_scan_incl_f64(tb);
#pragma unroll
    for (int k = 0; k < CPT; ++k) sq[k] += wb - tb;
    lds_store_own_f64<CPT>(Qb, sq);
    if (lane == 63) wQ[wv] = wb;
    __syncthreads();
    const double tq = lds_wave_values<NW>(wQ, lane, 0.0);
    const double iq = wave_scan_first_f64<NW>(tq);
    const double eq = iq - tq;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int n = nex[k];
      ps[k] = (sp[k] + offp) - (Qb[n] + shfl_f64(eq, n / SEG));
    }
  };

  // ---- parameters: log2-softmax of [0, theta] (extract_parameters.py:25-34)
  double pS[CPT], pD[CPT], pL[CPT], pT[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    pS[k] = pD[k] = pL[k] = pT[k] = 0.0;
    if (okp[k]) {
      const float* th = P.statewise ? P.theta + 3 * (size_t)colk[k] : P.theta;
      const double l0 = 0.0, l1 = th[0], l2 = th[1], l3 = th[2];
      const double mx = fmax(fmax(l0, l1), fmax(l2, l3));
      const double lse = mx + log2(exp2(l0 - mx) + exp2(l1 - mx) + exp2(l2 - mx) + exp2(l3 - mx));
      pS[k] = l0 - lse;
      pD[k] = l1 - lse;
      pL[k] = l2 - lse;
      pT[k] = l3 - lse;
    }
  }

  // ---- column log-probabilities and max_coupling
  double cl[CPT], mt[CPT], w[CPT];
  if (P.use_col) {
    // col_log_probs = log_softmax(col_weights) / ln2 (extract_parameters.py:37-38)
    double lmax = NINF;
#pragma unroll
    for (int k = 0; k < CPT; ++k)
      if (okp[k]) lmax = fmax(lmax, (double)P.col_weights[colk[k]]);
    const double gmax = block_max<NT>(lmax, red);
    double lsum = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k)
      if (okp[k]) lsum += exp((double)P.col_weights[colk[k]] - gmax);
    const double gsum = block_sum<NT>(lsum, red);
    const double lz = gmax + log(gsum);
    double pc[CPT], pcs[CPT], tot;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      cl[k] = okp[k] ? ((double)P.col_weights[colk[k]] - lz) / LN2 : 0.0;
      pc[k] = okp[k] ? exp2(cl[k]) : 0.0;
    }
    path_sums(pc, pcs, tot);
    // col_valid_log_normalizer (extract_parameters.py:41-65), then mt = pT + norm
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const double valid = 1.0 - pcs[k];
      const double cn = valid > 0.0 ? -log2(fmax(valid, 2.2250738585072014e-308)) : NINF;
      mt[k] = pT[k] + cn;
      w[k] = okp[k] ? exp2(cl[k]) : 0.0;
    }
  } else {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      cl[k] = -log2((double)S);
      mt[k] = okp[k] ? pT[k] + (double)P.unnorm_row_max[colk[k]] : 0.0;
      w[k] = okp[k] ? 1.0 : 0.0;
    }
  }

  // ---- E fixed point (pristine e_step.py:438-501) in linear float64
  double lin_pS[CPT], lin_pD[CPT], lin_pL[CPT], lin_mt[CPT], e[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    lin_pS[k] = exp2(pS[k]);
    lin_pD[k] = exp2(pD[k]);
    lin_pL[k] = exp2(pL[k]);
    lin_mt[k] = exp2(mt[k]);
    e[k] = okp[k] ? exp2(P.e_init) : 0.0;
  }
  const double ratio_hi = exp2(P.tol), ratio_lo = exp2(-P.tol);
  int it = 0;
  bool ok_local = true;  // convergence of the last update at the own positions
  double ps[CPT], e1[CPT], e2[CPT], rowsum = 0.0;
  for (;;) {
    // phase A: publish e and w e; inclusive preorder scan in registers; the
    // previous update's convergence flags
    double x[CPT], sp[CPT], ta = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      x[k] = w[k] * e[k];
      ta += x[k];
      sp[k] = ta;
    }
    const double wa = wave_scan_incl_f64(ta);
    lds_store_own_f64<CPT>(Eb, e);
    lds_store_own_f64<CPT>(Xw, x);
    const bool wave_ok = __ballot(!ok_local) == 0;
    if (lane == 63) {
      wP[wv] = wa;
      wok[wv] = wave_ok ? 1 : 0;
    }
    __syncthreads();
    // phase B: stop test, row sum and preorder offsets, postorder and child
    // gathers, exclusive postorder scan
    const int fl = lds_wave_values<NW>(wok, lane, 1);
    const bool all_ok = __ballot(fl == 0) == 0;
    const bool stop = it > 0 && (all_ok || it >= P.max_iter);
    const double tp = lds_wave_values<NW>(wP, lane, 0.0);
    double yq[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      yq[k] = Xw[qp[k]];
      e2[k] = Eb[c2p[k]];
    }
    const double e1last = Eb[c1last];
#pragma unroll
    for (int k = 0; k < CPT; ++k) e1[k] = k + 1 < CPT ? (h1[k] ? e[k + 1] : 0.0) : e1last;
    const double ip = wave_scan_first_f64<NW>(tp);
    rowsum = lane_value_f64(ip, NW - 1);
    const double offp = lane_value_f64(ip - tp, wv) + (wa - ta);
    double sq[CPT], tb = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      sq[k] = tb;
      tb += yq[k];
    }
    const double wb = wave_scan_incl_f64(tb);
#pragma unroll
    for (int k = 0; k < CPT; ++k) sq[k] += wb - tb;
    lds_store_own_f64<CPT>(Qb, sq);
    if (lane == 63) wQ[wv] = wb;
    __syncthreads();
    // phase C: path sums, then the update
    const double tq = lds_wave_values<NW>(wQ, lane, 0.0);
    const double iq = wave_scan_first_f64<NW>(tq);
    const double eq = iq - tq;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int n = nex[k];
      ps[k] = (sp[k] + offp) - (Qb[n] + shfl_f64(eq, n / SEG));
    }
    if (stop) break;
    ok_local = true;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      if (okp[k]) {
        const double na = rowsum - ps[k];
        const double eb = na > 0.0 ? lin_mt[k] * na : 0.0;
        const double en = lin_pS[k] * e1[k] * e2[k] + lin_pD[k] * e[k] * e[k] + e[k] * eb + lin_pL[k];
        // |log2(en / e)| < tol without a log or a division (e > 0):
        // en / e inside (2^-tol, 2^tol)
        if (!(en < e[k] * ratio_hi && en > e[k] * ratio_lo)) ok_local = false;
        e[k] = en;
      }
    }
    ++it;
  }
  if (tid == 0 && P.n_iter_out) P.n_iter_out[0] = it;

  // ---- outputs from the final E (pristine e_step.py:495-499)
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    if (!okp[k]) continue;
    const int s = colk[k];
    const int i = tid * CPT + k;
    const double E = log2(e[k]);
    const double Es1 = h1[k] ? log2(e1[k]) : NINF;
    const double Es2 = c2p[k] != ZERO ? log2(e2[k]) : NINF;
    const double na = rowsum - ps[k];
    const double Ebar = na > 0.0 ? log2(na) + mt[k] : NINF;
    P.E[s] = (float)E;
    P.E_s1[s] = (float)Es1;
    P.E_s2[s] = (float)Es2;
    P.Ebar[s] = (float)Ebar;
    if (P.E64) P.E64[s] = E;
    P.mt[s] = (float)mt[k];
    P.col_log_probs[s] = (float)cl[k];
    if (P.statewise) {
      P.log_pS[s] = (float)pS[k];
      P.log_pD[s] = (float)pD[k];
      P.log_pL[s] = (float)pL[k];
    } else if (s == 0) {
      P.log_pS[0] = (float)pS[k];
      P.log_pD[0] = (float)pD[k];
      P.log_pL[0] = (float)pL[k];
    }
    // row-kernel constants at preorder positions
    P.c_DL[i] = (float)(1.0 + pD[k] + E);
    P.c_SL1[i] = (float)(pS[k] + Es2);
    P.c_SL2[i] = (float)(pS[k] + Es1);
    P.c_pS[i] = (float)pS[k];
    P.c_pD[i] = (float)pD[k];
    P.c_colw[i] = (float)w[k];
    P.c_Ebar[i] = (float)Ebar;
    P.c_E[i] = (float)E;
    P.c_mt[i] = (float)mt[k];
    P.c_col[i] = (float)cl[k];
    P.lin_a[i] = (float)(exp2(1.0 + pD[k] + E) + exp2(Ebar));
    P.lin_emc[i] = (float)exp2(E + mt[k]);
    P.lin_k1[i] = (float)exp2(pS[k] + Es2);
    P.lin_k2[i] = (float)exp2(pS[k] + Es1);
  }
}

// Per-family loss term (solver.py:132-139):
//   -(LSE2(Pi[root]) - log2 S - log2(max(1 - mean(2^E), tiny)))
// One workgroup per family; the family sum is done by loss_sum_kernel in a
// fixed order, so the loss is bitwise reproducible.
constexpr int LNT = 256;
__global__ __launch_bounds__(LNT) void loss_terms_kernel(const float* pi, const int* root_rows, const float* E,
                                                         int S, double* terms) {
  __shared__ double red[LNT / 64];
  const int f = blockIdx.x;
  const float* row = pi + (size_t)root_rows[f] * S;
  double m = -__builtin_inf();
  for (int s = threadIdx.x; s < S; s += LNT) m = fmax(m, (double)row[s]);
  m = block_max<LNT>(m, red);
  double ms = m == -__builtin_inf() ? 0.0 : m;
  double acc = 0.0, eacc = 0.0;
  for (int s = threadIdx.x; s < S; s += LNT) {
    acc += exp2((double)row[s] - ms);
    eacc += exp2((double)E[s]);
  }
  acc = block_sum<LNT>(acc, red);
  eacc = block_sum<LNT>(eacc, red);
  if (threadIdx.x == 0) {
    double lse = acc > 0.0 ? log2(acc) + m : -__builtin_inf();
    double norm = fmax(1.0 - eacc / (double)S, 2.2250738585072014e-308);
    terms[f] = -(lse - log2((double)S) - log2(norm));
  }
}

__global__ __launch_bounds__(LNT) void loss_sum_kernel(const double* terms, int n, double* loss64, float* loss32) {
  __shared__ double red[LNT / 64];
  // fixed-order: each thread sums a contiguous chunk, then a fixed tree
  int chunk = (n + LNT - 1) / LNT;
  double acc = 0.0;
  for (int i = threadIdx.x * chunk; i < min(n, (int)(threadIdx.x + 1) * chunk); ++i) acc += terms[i];
  acc = block_sum<LNT>(acc, red);
  if (threadIdx.x == 0) {
    if (loss64) loss64[0] = acc;
    if (loss32) loss32[0] = (float)acc;
  }
}

void launch_estep(const EStepParams& P, hipStream_t st) {
  if (P.S <= 2048 && P.pd.post)
    hipLaunchKernelGGL((estep_pre_kernel<1024, 2>), dim3(1), dim3(1024), 0, st, P);
  else if (P.S <= 2048)
    hipLaunchKernelGGL(estep_fixed_point_kernel<2048>, dim3(1), dim3(ENT), 0, st, P);
  else
    hipLaunchKernelGGL(estep_fixed_point_kernel<8192>, dim3(1), dim3(ENT), 0, st, P);
}

void launch_loss(const float* pi, const int* root_rows, const float* E, int S, int n_fam, double* terms,
                 double* loss64, float* loss32, hipStream_t st) {
  hipLaunchKernelGGL(loss_terms_kernel, dim3(n_fam), dim3(LNT), 0, st, pi, root_rows, E, S, terms);
  hipLaunchKernelGGL(loss_sum_kernel, dim3(1), dim3(LNT), 0, st, terms, n_fam, loss64, loss32);
}

}  // namespace kb
