// Backward epilogue: E adjoint and the theta / column VJP, one workgroup, float64.
//
// Reference: kbench/api/_implicit_grad.py:373-475 (_e_adjoint_and_theta_vjp)
// with _bicgstab (_implicit_grad.py:28-94) and the E-step VJP kernels
// (pristine e_step.py:102-241), then autograd through
// extract_parameters_weighted_cols (extract_parameters.py:68-93).
//
// The E-step VJP is linear in its cotangents once E* is fixed, so the
// weights 2^(t_k - E_new), r = 2^(E - rowmax) and 1/denom are computed once;
// each BiCGSTAB mat-vec is then a child gather plus one subtree sum.
#include "kb_device.hpp"
#include "kb_kernels.hpp"

namespace kb {

constexpr int XNT = 1024;

struct EpiCtx {
  const EpiParams* P;
  double* red;
  double* X;      // LDS [S]
  double* U;      // LDS [S]
  double* scan2;  // LDS [2S] (Euler / preorder scans), null: sums by levels
};

__device__ __forceinline__ void levels_path_inplace(const EpiParams& P, double* v) {
  for (int d = 1; d < P.n_tlevels; ++d) {
    const int b = P.tlevel_ptr[d], e = P.tlevel_ptr[d + 1];
    for (int i = b + threadIdx.x; i < e; i += XNT) {
      const int n = P.tlevel_node[i];
      v[n] += v[P.tr.parent[n]];
    }
    __syncthreads();
  }
}

__device__ __forceinline__ void levels_subtree_inplace(const EpiParams& P, double* u) {
  for (int lv = 0; lv < P.tr.n_blevels; ++lv) {
    const int b = P.tr.blevel_ptr[lv], e = P.tr.blevel_ptr[lv + 1];
    for (int i = b + threadIdx.x; i < e; i += XNT) {
      const int p = P.tr.blevel_node[i];
      const int x = P.tr.c1[p], y = P.tr.c2[p];
      u[p] += (x >= 0 ? u[x] : 0.0) + (y >= 0 ? u[y] : 0.0);
    }
    __syncthreads();
  }
}

__device__ __forceinline__ void path_inplace(const EpiCtx& c, double* v) {
  if (c.scan2)
    euler_path_sums_f64<1024>(c.P->ts, v, c.scan2, c.red);
  else
    levels_path_inplace(*c.P, v);
}

__device__ __forceinline__ void subtree_inplace(const EpiCtx& c, double* u) {
  if (c.scan2)
    preorder_subtree_sums_f64<1024>(c.P->ts, u, c.scan2, c.red);
  else
    levels_subtree_inplace(*c.P, u);
}

// work-vector slots ([S] float64 each)
enum {
  W_W0, W_W1, W_W2, W_W3, W_R, W_ID, W_E,
  V_X, V_R, V_RH, V_V, V_P, V_S, V_T, V_TMP, V_Q, N_WORK
};

__device__ __forceinline__ double* wv(const EpiParams& P, int slot) { return P.work + (size_t)slot * P.S; }

// gE = VJP of E_new / (E_s1, E_s2, Ebar) outputs w.r.t. E (pristine e_step.py:164-241).
// gnew, gs1, gs2, gebar may be null (zero).  Optional col_out gets r (tot - excl).
__device__ void estep_vjp(const EpiCtx& c, const double* gnew, const double* gs1, const double* gs2,
                          const double* gebar, double* gE, double* q0_out, double* q1_out, double* q3_out,
                          double* wbar_out, double* col_out) {
  const EpiParams& P = *c.P;
  const int S = P.S;
  const double* W0 = wv(P, W_W0);
  const double* W1 = wv(P, W_W1);
  const double* W2 = wv(P, W_W2);
  const double* W3 = wv(P, W_W3);
  const double* R = wv(P, W_R);
  const double* ID = wv(P, W_ID);
  // q0 + gs1 to LDS (gathered by c1-children)
  for (int s = threadIdx.x; s < S; s += XNT) {
    const double g = gnew ? gnew[s] : 0.0;
    const double q0 = g * W0[s];
    c.X[s] = q0 + (gs1 ? gs1[s] : 0.0);
    c.U[s] = q0 + (gs2 ? gs2[s] : 0.0);
  }
  __syncthreads();
  double lu = 0.0;
  for (int s = threadIdx.x; s < S; s += XNT) {
    const double g = gnew ? gnew[s] : 0.0;
    const double q1 = g * W1[s], q2 = g * W2[s];
    double acc = 2.0 * q1 + q2;
    const int p = P.tr.parent[s];
    if (p >= 0) acc += (P.tr.c1[p] == s) ? c.X[p] : c.U[p];
    gE[s] = acc;
    const double wbar = q2 + (gebar ? gebar[s] : 0.0);
    if (q0_out) q0_out[s] = g * W0[s];
    if (q1_out) q1_out[s] = q1;
    if (q3_out) q3_out[s] = g * W3[s];
    if (wbar_out) wbar_out[s] = wbar;
    lu += wbar * ID[s];
  }
  __syncthreads();
  const double tot = block_sum<XNT>(lu, c.red);
  for (int s = threadIdx.x; s < S; s += XNT) {
    const double g = gnew ? gnew[s] : 0.0;
    c.U[s] = (g * W2[s] + (gebar ? gebar[s] : 0.0)) * ID[s];
  }
  __syncthreads();
  subtree_inplace(c, c.U);
  for (int s = threadIdx.x; s < S; s += XNT) {
    const double pv = R[s] * (tot - c.U[s]);
    gE[s] += pv;
    if (col_out) col_out[s] = pv;
  }
  __syncthreads();
}

__device__ __forceinline__ double dot(const EpiCtx& c, const double* a, const double* b) {
  double l = 0.0;
  for (int s = threadIdx.x; s < c.P->S; s += XNT) l += a[s] * b[s];
  return block_sum<XNT>(l, c.red);
}

// y = x - J^T x
__device__ __forceinline__ void ag(const EpiCtx& c, const double* x, double* y) {
  estep_vjp(c, x, nullptr, nullptr, nullptr, y, nullptr, nullptr, nullptr, nullptr, nullptr);
  for (int s = threadIdx.x; s < c.P->S; s += XNT) y[s] = x[s] - y[s];
  __syncthreads();
}

template <int MAXS>
__global__ __launch_bounds__(XNT) void epilogue_kernel(EpiParams P) {
  __shared__ double X[MAXS];
  __shared__ double U[MAXS];
  __shared__ double red[XNT / 64];
  __shared__ double scan2[MAXS <= 4096 ? 2 * MAXS : 1];
  EpiCtx c{&P, red, X, U, MAXS <= 4096 ? scan2 : nullptr};
  const int S = P.S;
  const int tid = threadIdx.x;
  const double NINF = -__builtin_inf();
  const double TINY = 2.2250738585072014e-308;
  const double LN2 = 0.6931471805599453;
  const double* acc = P.acc;
  const double* a_pD = acc + 0 * (size_t)S;
  const double* a_pS = acc + 1 * (size_t)S;
  const double* a_E = acc + 2 * (size_t)S;
  const double* a_Ebar = acc + 3 * (size_t)S;
  const double* a_Es1 = acc + 4 * (size_t)S;
  const double* a_Es2 = acc + 5 * (size_t)S;
  const double* a_mt = acc + 6 * (size_t)S;
  const double* a_col = acc + 7 * (size_t)S;
  double* Ev = wv(P, W_E);

  // ---- E-step linearisation at E* (fp64 recomputation of pristine e_step.py:42-91)
  double lm = NINF;
  for (int s = tid; s < S; s += XNT) {
    const double e = (double)P.E[s];
    Ev[s] = e;
    X[s] = e;
    lm = fmax(lm, P.use_col ? (double)P.col[s] + e : e);
  }
  const double rmax = block_max<XNT>(lm, red);  // publishes X
  const double rms = rmax == NINF ? 0.0 : rmax;
  double ls = 0.0;
  for (int s = tid; s < S; s += XNT) {
    const double r = exp2((P.use_col ? (double)P.col[s] + X[s] : X[s]) - rms);
    wv(P, W_R)[s] = r;
    U[s] = r;
    ls += r;
  }
  const double rowsum = block_sum<XNT>(ls, red);
  path_inplace(c, U);
  for (int s = tid; s < S; s += XNT) {
    const int a1 = P.tr.c1[s], a2 = P.tr.c2[s];
    const double E = X[s];
    const double Es1 = a1 >= 0 ? X[a1] : NINF, Es2 = a2 >= 0 ? X[a2] : NINF;
    const double denom = rowsum - U[s];
    const double Ebar = denom > 0.0 ? log2(denom) + rmax + (double)P.mt[s] : NINF;
    wv(P, W_ID)[s] = denom > 0.0 ? 1.0 / denom : 0.0;
    const double pS = P.log_pS[P.statewise ? s : 0], pD = P.log_pD[P.statewise ? s : 0];
    const double pL = P.log_pL[P.statewise ? s : 0];
    const double t0 = pS + Es1 + Es2, t1 = pD + 2.0 * E, t2 = E + Ebar, t3 = pL;
    const double m = fmax(fmax(t0, t1), fmax(t2, t3));
    const double ms = m == NINF ? 0.0 : m;
    const double En = log2(exp2(t0 - ms) + exp2(t1 - ms) + exp2(t2 - ms) + exp2(t3 - ms)) + m;
    auto wgt = [&](double t) {
      double w = exp2(t - En);
      return (w == w) ? w : 0.0;  // NaN (both -inf) -> 0
    };
    wv(P, W_W0)[s] = wgt(t0);
    wv(P, W_W1)[s] = wgt(t1);
    wv(P, W_W2)[s] = wgt(t2);
    wv(P, W_W3)[s] = wgt(t3);
  }
  __syncthreads();

  // ---- q_E = grad_E + d/dE [n_fam log2(norm) + <E_s1,gEs1> + <E_s2,gEs2> + <Ebar,gEbar>]
  double le = 0.0;
  for (int s = tid; s < S; s += XNT) le += exp2(Ev[s]);
  const double mean = block_sum<XNT>(le, red) / (double)S;
  const double norm = 1.0 - mean;
  const double scale = (P.n_items_rows == P.n_fam) ? 1.0 : (double)P.n_fam;
  double* qE = wv(P, V_Q);
  estep_vjp(c, nullptr, a_Es1, a_Es2, a_Ebar, qE, nullptr, nullptr, nullptr, nullptr, nullptr);
  for (int s = tid; s < S; s += XNT) {
    const double dd = (!P.no_norm && norm >= TINY) ? -scale * exp2(Ev[s]) / ((double)S * norm) : 0.0;
    qE[s] = a_E[s] + qE[s] + dd + (P.q_extra ? P.q_extra[s] : 0.0);
  }
  __syncthreads();

  // ---- BiCGSTAB on (I - J^T) w = q_E (_implicit_grad.py:28-94, same stopping rules)
  double* x = wv(P, V_X);
  double* r = wv(P, V_R);
  double* rh = wv(P, V_RH);
  double* vv = wv(P, V_V);
  double* pp = wv(P, V_P);
  double* sv = wv(P, V_S);
  double* tv = wv(P, V_T);
  double* tmp = wv(P, V_TMP);
  for (int s = tid; s < S; s += XNT) x[s] = 0.0;
  __syncthreads();
  ag(c, x, tmp);
  for (int s = tid; s < S; s += XNT) r[s] = qE[s] - tmp[s];
  __syncthreads();
  const double bnorm = fmax(sqrt(dot(c, qE, qE)), 1.0);
  double rel = sqrt(dot(c, r, r)) / bnorm;
  int k = 0;
  int done = rel <= P.tol;
  int failed = 0;
  double* wsol = x;
  if (!done) {
    for (int s = tid; s < S; s += XNT) {
      rh[s] = r[s];
      vv[s] = 0.0;
      pp[s] = 0.0;
    }
    __syncthreads();
    double rho_old = 1.0, alpha = 1.0, omega = 1.0;
    for (k = 1; k <= P.max_iter; ++k) {
      const double rho = dot(c, rh, r);
      if (fabs(rho) <= P.breakdown) break;
      const double beta = (rho / rho_old) * (alpha / omega);
      for (int s = tid; s < S; s += XNT) pp[s] = r[s] + beta * (pp[s] - omega * vv[s]);
      __syncthreads();
      ag(c, pp, vv);
      const double den = dot(c, rh, vv);
      if (fabs(den) <= P.breakdown) break;
      alpha = rho / den;
      for (int s = tid; s < S; s += XNT) sv[s] = r[s] - alpha * vv[s];
      __syncthreads();
      if (sqrt(dot(c, sv, sv)) / bnorm <= P.tol) {
        for (int s = tid; s < S; s += XNT) tmp[s] = x[s] + alpha * pp[s];
        __syncthreads();
        wsol = tmp;
        done = 1;
        break;
      }
      ag(c, sv, tv);
      const double tt = dot(c, tv, tv);
      if (fabs(tt) <= P.breakdown) break;
      omega = dot(c, tv, sv) / tt;
      for (int s = tid; s < S; s += XNT) {
        x[s] = x[s] + alpha * pp[s] + omega * sv[s];
        r[s] = sv[s] - omega * tv[s];
      }
      __syncthreads();
      rel = sqrt(dot(c, r, r)) / bnorm;
      if (rel <= P.tol) {
        done = 1;
        break;
      }
      if (fabs(omega) <= P.breakdown) break;
      rho_old = rho;
    }
    if (!done) failed = 1;
    if (k > P.max_iter) k = P.max_iter;
  }
  if (tid == 0) {
    P.status[0] = k;
    P.status[1] = failed;
  }

  // ---- parameter cotangents: param_loss + E-step(E*, params) with (wE, g_Ebar)
  double* G_pS = wv(P, V_R);
  double* G_pD = wv(P, V_RH);
  double* G_pL = wv(P, V_V);
  double* G_mt = wv(P, V_P);
  double* G_col = wv(P, V_S);
  double* gE_dummy = wv(P, V_T);
  if (wsol != tmp) {
    for (int s = tid; s < S; s += XNT) tmp[s] = wsol[s];
    __syncthreads();
  }
  estep_vjp(c, tmp, nullptr, nullptr, a_Ebar, gE_dummy, G_pS, G_pD, G_pL, G_mt, G_col);
  for (int s = tid; s < S; s += XNT) {
    G_pS[s] += a_pS[s];
    G_pD[s] += a_pD[s];
    G_mt[s] += a_mt[s];
    G_col[s] += a_col[s];
  }
  __syncthreads();
  if (P.g_out) {  // E adjoint and per-state parameter cotangents only
    for (int s = tid; s < S; s += XNT) {
      P.g_out[s] = G_pS[s];
      P.g_out[(size_t)S + s] = G_pD[s];
      P.g_out[2 * (size_t)S + s] = G_pL[s];
      P.g_out[3 * (size_t)S + s] = G_mt[s];
      P.g_out[4 * (size_t)S + s] = G_col[s];
      if (P.w_out) P.w_out[s] = tmp[s];
    }
    return;
  }

  // theta VJP through log2-softmax of [0, theta] (extract_parameters.py:71-74)
  if (P.statewise) {
    for (int s = tid; s < S; s += XNT) {
      const float* th = P.theta + 3 * (size_t)s;
      const double l0 = 0.0, l1 = th[0], l2 = th[1], l3 = th[2];
      const double mx = fmax(fmax(l0, l1), fmax(l2, l3));
      const double z = exp2(l0 - mx) + exp2(l1 - mx) + exp2(l2 - mx) + exp2(l3 - mx);
      const double gs = G_pS[s] + G_pD[s] + G_pL[s] + G_mt[s];
      P.grad_theta[3 * (size_t)s + 0] = (float)(G_pD[s] - exp2(l1 - mx) / z * gs);
      P.grad_theta[3 * (size_t)s + 1] = (float)(G_pL[s] - exp2(l2 - mx) / z * gs);
      P.grad_theta[3 * (size_t)s + 2] = (float)(G_mt[s] - exp2(l3 - mx) / z * gs);
    }
  } else {
    double a = 0.0, b = 0.0, d = 0.0, e = 0.0;
    for (int s = tid; s < S; s += XNT) {
      a += G_pS[s];
      b += G_pD[s];
      d += G_pL[s];
      e += G_mt[s];
    }
    a = block_sum<XNT>(a, red);
    b = block_sum<XNT>(b, red);
    d = block_sum<XNT>(d, red);
    e = block_sum<XNT>(e, red);
    if (tid == 0) {
      const double l0 = 0.0, l1 = P.theta[0], l2 = P.theta[1], l3 = P.theta[2];
      const double mx = fmax(fmax(l0, l1), fmax(l2, l3));
      const double z = exp2(l0 - mx) + exp2(l1 - mx) + exp2(l2 - mx) + exp2(l3 - mx);
      const double gs = a + b + d + e;
      P.grad_theta[0] = (float)(b - exp2(l1 - mx) / z * gs);
      P.grad_theta[1] = (float)(d - exp2(l2 - mx) / z * gs);
      P.grad_theta[2] = (float)(e - exp2(l3 - mx) / z * gs);
    }
  }

  // column VJP: col_log_probs = log_softmax(w)/ln2, col_norm = -log2(1 - pathsum(2^cl))
  double lmx = NINF;
  for (int s = tid; s < S; s += XNT) lmx = fmax(lmx, (double)P.col_weights[s]);
  const double wmax = block_max<XNT>(lmx, red);
  double lz = 0.0;
  for (int s = tid; s < S; s += XNT) lz += exp((double)P.col_weights[s] - wmax);
  const double zsum = block_sum<XNT>(lz, red);
  const double logz = wmax + log(zsum);
  for (int s = tid; s < S; s += XNT) U[s] = exp2(((double)P.col_weights[s] - logz) / LN2);
  __syncthreads();
  path_inplace(c, U);
  for (int s = tid; s < S; s += XNT) {
    const double valid = 1.0 - U[s];
    X[s] = (valid > 0.0 && valid >= TINY) ? G_mt[s] / valid : 0.0;
  }
  __syncthreads();
  subtree_inplace(c, X);
  double lg = 0.0;
  for (int s = tid; s < S; s += XNT) {
    const double pc = exp2(((double)P.col_weights[s] - logz) / LN2);
    const double g = G_col[s] + pc * X[s];
    tmp[s] = g;
    lg += g;
  }
  const double gsum = block_sum<XNT>(lg, red);  // publishes tmp
  for (int s = tid; s < S; s += XNT) {
    const double qn = exp((double)P.col_weights[s] - logz);
    P.grad_col[s] = (float)((tmp[s] - qn * gsum) / LN2);
  }
}

// ---- register-resident epilogue for trees of up to NT*CPT nodes ------------
// The algorithm, the order of the BiCGSTAB steps and the stopping rules are
// those of epilogue_kernel above; every [S] vector lives in registers at
// preorder positions (thread t owns positions t*CPT + k), and the sums over
// the tree are register scans (DPP float64) with one LDS exchange:
//   * one E-step VJP (a parent gather and one subtree sum): one barrier;
//   * one or two dot products: one barrier;
//   * ancestors-or-self sums, Pre(i) - PostEx(tin(i) - i): two barriers.
template <int NT, int CPT>
__global__ __launch_bounds__(NT) void epilogue_pre_kernel(EpiParams P) {
  constexpr int MAXS = NT * CPT;
  constexpr int NW = NT / 64;
  constexpr int ZERO = MAXS;     // padding slot: 0 in every buffer
  constexpr int SEG = 64 * CPT;  // positions / postorder slots per wavefront
  __shared__ __align__(16) double Xp[MAXS + 64];  // VJP: child1-side values for the parent gather
  __shared__ __align__(16) double Up[MAXS + 64];  // VJP: child2-side values; E for the child gathers
  __shared__ __align__(16) double Lv[MAXS + 64];  // wavefront-local inclusive preorder scan
  __shared__ __align__(16) double Xw[MAXS + 64];  // path sums: values at positions
  __shared__ __align__(16) double Qb[MAXS + 64];  // path sums: wavefront-local exclusive postorder scan
  __shared__ double wV[NW], wP[NW], wQ[NW], mred[NW];
  __shared__ double red[2][2 * NW];
  const PreDev& T = P.pd;
  const int S = P.S;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const double NINF = -__builtin_inf();
  const double TINY = 2.2250738585072014e-308;
  const double LN2 = 0.6931471805599453;

  int colk[CPT], c2p[CPT], nex[CPT], qp[CPT], ppos[CPT], endm1[CPT];
  bool okp[CPT], h1[CPT], pfl[CPT];
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
    const int pa = okp[k] ? T.ppos[i] : -1;
    ppos[k] = pa >= 0 ? pa : ZERO;
    pfl[k] = pa >= 0 && T.pflag[i] != 0;
    endm1[k] = okp[k] ? T.endpos[i] - 1 : ZERO;
  }
  const int c1last = h1[CPT - 1] ? tid * CPT + CPT : ZERO;
  if (tid < 64) {
    Xp[MAXS + tid] = 0.0;
    Up[MAXS + tid] = 0.0;
    Lv[MAXS + tid] = 0.0;
    Xw[MAXS + tid] = 0.0;
    Qb[MAXS + tid] = 0.0;
  }
  __syncthreads();

  // sums over all positions of a and b (fixed order), one barrier
  int rbuf = 0;
  auto sum2 = [&](double a, double b, double& ra, double& rb) {
    const double sa = lane_value_f64(wave_scan_incl_f64(a), 63);
    const double sb = lane_value_f64(wave_scan_incl_f64(b), 63);
    double* R = red[rbuf];
    rbuf ^= 1;
    if (lane == 0) {
      R[wv] = sa;
      R[NW + wv] = sb;
    }
    __syncthreads();
    ra = 0.0;
    rb = 0.0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      ra += R[w];
      rb += R[NW + w];
    }
  };
  auto dot = [&](const double (&a)[CPT], const double (&b)[CPT]) {
    double l = 0.0, r0, r1;
#pragma unroll
    for (int k = 0; k < CPT; ++k) l += a[k] * b[k];
    sum2(l, 0.0, r0, r1);
    return r0;
  };

  // ancestors-or-self sums of x and the total (two barriers)
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

  // subtree (descendants-or-self) sums of u after the caller's scan setup:
  // sc = wavefront-local inclusive scan (published in Lv with the wavefront
  // totals in wV before the caller's barrier); returns the total
  auto subtree_finish = [&](const double (&sc)[CPT], double (&sub)[CPT]) {
    double le[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) le[k] = Lv[endm1[k]];
    const double tv = lds_wave_values<NW>(wV, lane, 0.0);
    const double iv = wave_scan_first_f64<NW>(tv);
    const double ev = iv - tv;
    const double tot = lane_value_f64(iv, NW - 1);
    const double offv = lane_value_f64(ev, wv);
    const double pm0 = wave_prev_lane_f64(sc[CPT - 1]) + offv;  // P[i - 1] of slot 0
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const double pm1 = k == 0 ? pm0 : sc[k - 1] + offv;
      sub[k] = (le[k] + shfl_f64(ev, endm1[k] / SEG)) - pm1;
    }
    return tot;
  };

  // ---- E-step linearisation at E* (fp64 recomputation of pristine e_step.py:42-91)
  double Ev[CPT], R[CPT], ID[CPT], W0[CPT], W1[CPT], W2[CPT], W3[CPT];
  double lm = NINF;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    Ev[k] = okp[k] ? (double)P.E[colk[k]] : 0.0;
    if (okp[k]) lm = fmax(lm, P.use_col ? (double)P.col[colk[k]] + Ev[k] : Ev[k]);
  }
  lds_store_own_f64<CPT>(Up, Ev);  // for the child gathers (published by the barriers below)
  const double rmax = block_max<NT>(lm, mred);
  const double rms = rmax == NINF ? 0.0 : rmax;
#pragma unroll
  for (int k = 0; k < CPT; ++k)
    R[k] = okp[k] ? exp2((P.use_col ? (double)P.col[colk[k]] + Ev[k] : Ev[k]) - rms) : 0.0;
  double Upath[CPT], rowsum;
  path_sums(R, Upath, rowsum);
  {
    const double e1last = Up[c1last];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      W0[k] = W1[k] = W2[k] = W3[k] = ID[k] = 0.0;
      if (!okp[k]) continue;
      const int s = colk[k];
      const double E = Ev[k];
      const double Es1 = h1[k] ? (k + 1 < CPT ? Ev[k + 1] : e1last) : NINF;
      const double Es2 = c2p[k] != ZERO ? Up[c2p[k]] : NINF;
      const double denom = rowsum - Upath[k];
      const double Ebar = denom > 0.0 ? log2(denom) + rmax + (double)P.mt[s] : NINF;
      ID[k] = denom > 0.0 ? 1.0 / denom : 0.0;
      const double pS = P.log_pS[P.statewise ? s : 0], pD = P.log_pD[P.statewise ? s : 0];
      const double pL = P.log_pL[P.statewise ? s : 0];
      const double t0 = pS + Es1 + Es2, t1 = pD + 2.0 * E, t2 = E + Ebar, t3 = pL;
      const double m = fmax(fmax(t0, t1), fmax(t2, t3));
      const double ms = m == NINF ? 0.0 : m;
      const double En = log2(exp2(t0 - ms) + exp2(t1 - ms) + exp2(t2 - ms) + exp2(t3 - ms)) + m;
      auto wgt = [&](double t) {
        double w = exp2(t - En);
        return (w == w) ? w : 0.0;  // NaN (both -inf) -> 0
      };
      W0[k] = wgt(t0);
      W1[k] = wgt(t1);
      W2[k] = wgt(t2);
      W3[k] = wgt(t3);
    }
  }

  // E-step VJP (pristine e_step.py:164-241) at the own positions, one barrier:
  //   q_j = g W_j, wbar = q2 + gebar, tot = sum wbar ID,
  //   gE = 2 q1 + q2 + (parent's q0 + gs1 if child1, else q0 + gs2) + R (tot - subtree(wbar ID)).
  // gs1 / gs2 / gebar are column-indexed (may be null); pv = R (tot - subtree).
  auto vjp = [&](const double (&g)[CPT], const double* gs1, const double* gs2, const double* gebar,
                 double (&gE)[CPT], double (&wbar)[CPT], double (&pv)[CPT]) {
    double xo[CPT], uo[CPT], sc[CPT], ta = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = colk[k];
      const double q0 = g[k] * W0[k];
      xo[k] = q0 + ((gs1 && okp[k]) ? gs1[s] : 0.0);
      uo[k] = q0 + ((gs2 && okp[k]) ? gs2[s] : 0.0);
      wbar[k] = g[k] * W2[k] + ((gebar && okp[k]) ? gebar[s] : 0.0);
      ta += wbar[k] * ID[k];
      sc[k] = ta;
    }
    const double wa = wave_scan_incl_f64(ta);
#pragma unroll
    for (int k = 0; k < CPT; ++k) sc[k] += wa - ta;
    lds_store_own_f64<CPT>(Xp, xo);
    lds_store_own_f64<CPT>(Up, uo);
    lds_store_own_f64<CPT>(Lv, sc);
    if (lane == 63) wV[wv] = wa;
    __syncthreads();
    double par[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) par[k] = pfl[k] ? Xp[ppos[k]] : Up[ppos[k]];  // root: padding 0
    double sub[CPT];
    const double tot = subtree_finish(sc, sub);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const double q1 = g[k] * W1[k], q2 = g[k] * W2[k];
      double acc = 2.0 * q1 + q2;
      acc += par[k];
      const double p = R[k] * (tot - sub[k]);
      gE[k] = acc + p;
      pv[k] = p;
    }
  };
  // y = x - J^T x
  auto ag = [&](const double (&xv)[CPT], double (&y)[CPT]) {
    double gE[CPT], wb[CPT], pv[CPT];
    vjp(xv, nullptr, nullptr, nullptr, gE, wb, pv);
#pragma unroll
    for (int k = 0; k < CPT; ++k) y[k] = xv[k] - gE[k];
  };

  const double* acc = P.acc;
  const double* a_pD = acc + 0 * (size_t)S;
  const double* a_pS = acc + 1 * (size_t)S;
  const double* a_E = acc + 2 * (size_t)S;
  const double* a_Ebar = acc + 3 * (size_t)S;
  const double* a_Es1 = acc + 4 * (size_t)S;
  const double* a_Es2 = acc + 5 * (size_t)S;
  const double* a_mt = acc + 6 * (size_t)S;
  const double* a_col = acc + 7 * (size_t)S;

  // ---- q_E = grad_E + d/dE [n_fam log2(norm) + <E_s1,gEs1> + <E_s2,gEs2> + <Ebar,gEbar>]
  double qE[CPT];
  {
    double le = 0.0, r0, r1;
#pragma unroll
    for (int k = 0; k < CPT; ++k)
      if (okp[k]) le += exp2(Ev[k]);
    sum2(le, 0.0, r0, r1);
    const double mean = r0 / (double)S;
    const double norm = 1.0 - mean;
    const double scale = (P.n_items_rows == P.n_fam) ? 1.0 : (double)P.n_fam;
    double zero[CPT], gE[CPT], wb[CPT], pv[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) zero[k] = 0.0;
    vjp(zero, a_Es1, a_Es2, a_Ebar, gE, wb, pv);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const double dd = (!P.no_norm && norm >= TINY) ? -scale * exp2(Ev[k]) / ((double)S * norm) : 0.0;
      const double qx = (okp[k] && P.q_extra) ? P.q_extra[colk[k]] : 0.0;
      qE[k] = okp[k] ? a_E[colk[k]] + gE[k] + dd + qx : 0.0;
    }
  }

  // ---- BiCGSTAB on (I - J^T) w = q_E (_implicit_grad.py:28-94, same stopping rules).
  // A x with x = 0 is exactly 0, so r = q_E.
  double x[CPT], r[CPT], xs[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    x[k] = 0.0;
    r[k] = qE[k];
  }
  const double qq = dot(qE, qE);
  const double bnorm = fmax(sqrt(qq), 1.0);
  double rel = sqrt(qq) / bnorm;
  int kit = 0;
  int done = rel <= P.tol;
  int failed = 0;
  bool use_xs = false;
  if (!done) {
    double rh[CPT], vv[CPT], pp[CPT], sv[CPT], tv[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      rh[k] = r[k];
      vv[k] = 0.0;
      pp[k] = 0.0;
    }
    double rho_old = 1.0, alpha = 1.0, omega = 1.0, rho_next = 0.0;
    for (kit = 1; kit <= P.max_iter; ++kit) {
      const double rho = kit == 1 ? dot(rh, r) : rho_next;
      if (fabs(rho) <= P.breakdown) break;
      const double beta = (rho / rho_old) * (alpha / omega);
#pragma unroll
      for (int k = 0; k < CPT; ++k) pp[k] = r[k] + beta * (pp[k] - omega * vv[k]);
      ag(pp, vv);
      const double den = dot(rh, vv);
      if (fabs(den) <= P.breakdown) break;
      alpha = rho / den;
#pragma unroll
      for (int k = 0; k < CPT; ++k) sv[k] = r[k] - alpha * vv[k];
      if (sqrt(dot(sv, sv)) / bnorm <= P.tol) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) xs[k] = x[k] + alpha * pp[k];
        use_xs = true;
        done = 1;
        break;
      }
      ag(sv, tv);
      double tt, ts;
      {
        double lt = 0.0, ls = 0.0;
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
          lt += tv[k] * tv[k];
          ls += tv[k] * sv[k];
        }
        sum2(lt, ls, tt, ts);
      }
      if (fabs(tt) <= P.breakdown) break;
      omega = ts / tt;
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        x[k] = x[k] + alpha * pp[k] + omega * sv[k];
        r[k] = sv[k] - omega * tv[k];
      }
      double rr;
      {
        double lr = 0.0, lh = 0.0;
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
          lr += r[k] * r[k];
          lh += rh[k] * r[k];
        }
        sum2(lr, lh, rr, rho_next);
      }
      rel = sqrt(rr) / bnorm;
      if (rel <= P.tol) {
        done = 1;
        break;
      }
      if (fabs(omega) <= P.breakdown) break;
      rho_old = rho;
    }
    if (!done) failed = 1;
    if (kit > P.max_iter) kit = P.max_iter;
  }
  if (tid == 0) {
    P.status[0] = kit;
    P.status[1] = failed;
  }

  // ---- parameter cotangents: param_loss + E-step(E*, params) with (wE, g_Ebar)
  double G_pS[CPT], G_pD[CPT], G_pL[CPT], G_mt[CPT], G_col[CPT];
  {
    double ws[CPT], gE[CPT], wb[CPT], pv[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) ws[k] = use_xs ? xs[k] : x[k];
    vjp(ws, nullptr, nullptr, a_Ebar, gE, wb, pv);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = colk[k];
      G_pS[k] = okp[k] ? ws[k] * W0[k] + a_pS[s] : 0.0;
      G_pD[k] = okp[k] ? ws[k] * W1[k] + a_pD[s] : 0.0;
      G_pL[k] = okp[k] ? ws[k] * W3[k] : 0.0;
      G_mt[k] = okp[k] ? wb[k] + a_mt[s] : 0.0;
      G_col[k] = okp[k] ? pv[k] + a_col[s] : 0.0;
    }
    if (P.g_out) {  // E adjoint and per-state parameter cotangents only
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        if (!okp[k]) continue;
        const int s = colk[k];
        P.g_out[s] = G_pS[k];
        P.g_out[(size_t)S + s] = G_pD[k];
        P.g_out[2 * (size_t)S + s] = G_pL[k];
        P.g_out[3 * (size_t)S + s] = G_mt[k];
        P.g_out[4 * (size_t)S + s] = G_col[k];
        if (P.w_out) P.w_out[s] = ws[k];
      }
      return;
    }
  }

  // theta VJP through log2-softmax of [0, theta] (extract_parameters.py:71-74)
  if (P.statewise) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      if (!okp[k]) continue;
      const int s = colk[k];
      const float* th = P.theta + 3 * (size_t)s;
      const double l0 = 0.0, l1 = th[0], l2 = th[1], l3 = th[2];
      const double mx = fmax(fmax(l0, l1), fmax(l2, l3));
      const double z = exp2(l0 - mx) + exp2(l1 - mx) + exp2(l2 - mx) + exp2(l3 - mx);
      const double gs = G_pS[k] + G_pD[k] + G_pL[k] + G_mt[k];
      P.grad_theta[3 * (size_t)s + 0] = (float)(G_pD[k] - exp2(l1 - mx) / z * gs);
      P.grad_theta[3 * (size_t)s + 1] = (float)(G_pL[k] - exp2(l2 - mx) / z * gs);
      P.grad_theta[3 * (size_t)s + 2] = (float)(G_mt[k] - exp2(l3 - mx) / z * gs);
    }
  } else {
    double a = 0.0, b = 0.0, d = 0.0, e = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      a += G_pS[k];
      b += G_pD[k];
      d += G_pL[k];
      e += G_mt[k];
    }
    sum2(a, b, a, b);
    sum2(d, e, d, e);
    if (tid == 0) {
      const double l0 = 0.0, l1 = P.theta[0], l2 = P.theta[1], l3 = P.theta[2];
      const double mx = fmax(fmax(l0, l1), fmax(l2, l3));
      const double z = exp2(l0 - mx) + exp2(l1 - mx) + exp2(l2 - mx) + exp2(l3 - mx);
      const double gs = a + b + d + e;
      P.grad_theta[0] = (float)(b - exp2(l1 - mx) / z * gs);
      P.grad_theta[1] = (float)(d - exp2(l2 - mx) / z * gs);
      P.grad_theta[2] = (float)(e - exp2(l3 - mx) / z * gs);
    }
  }

  // column VJP: col_log_probs = log_softmax(w)/ln2, col_norm = -log2(1 - pathsum(2^cl))
  double lmx = NINF;
#pragma unroll
  for (int k = 0; k < CPT; ++k)
    if (okp[k]) lmx = fmax(lmx, (double)P.col_weights[colk[k]]);
  const double wmax = block_max<NT>(lmx, mred);
  double lz = 0.0;
#pragma unroll
  for (int k = 0; k < CPT; ++k)
    if (okp[k]) lz += exp((double)P.col_weights[colk[k]] - wmax);
  double zsum, unused;
  sum2(lz, 0.0, zsum, unused);
  const double logz = wmax + log(zsum);
  double pc[CPT], pcs[CPT], ptot;
#pragma unroll
  for (int k = 0; k < CPT; ++k) pc[k] = okp[k] ? exp2(((double)P.col_weights[colk[k]] - logz) / LN2) : 0.0;
  path_sums(pc, pcs, ptot);
  double sc[CPT], ta = 0.0;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const double valid = 1.0 - pcs[k];
    const double xv = (okp[k] && valid > 0.0 && valid >= TINY) ? G_mt[k] / valid : 0.0;
    ta += xv;
    sc[k] = ta;
  }
  const double wa = wave_scan_incl_f64(ta);
#pragma unroll
  for (int k = 0; k < CPT; ++k) sc[k] += wa - ta;
  lds_store_own_f64<CPT>(Lv, sc);
  if (lane == 63) wV[wv] = wa;
  __syncthreads();
  double sub[CPT];
  subtree_finish(sc, sub);
  double g[CPT], lg = 0.0;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    g[k] = okp[k] ? G_col[k] + pc[k] * sub[k] : 0.0;
    lg += g[k];
  }
  double gsum;
  sum2(lg, 0.0, gsum, unused);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    if (!okp[k]) continue;
    const int s = colk[k];
    const double qn = exp((double)P.col_weights[s] - logz);
    P.grad_col[s] = (float)((g[k] - qn * gsum) / LN2);
  }
}

void launch_epilogue(const EpiParams& P, hipStream_t st) {
  if (P.S <= 2048 && P.pd.post)  // 512 x 4: fewer wavefronts, less per-wavefront scan overhead
    hipLaunchKernelGGL((epilogue_pre_kernel<512, 4>), dim3(1), dim3(512), 0, st, P);
  else if (P.S <= 2048)
    hipLaunchKernelGGL(epilogue_kernel<2048>, dim3(1), dim3(XNT), 0, st, P);
  else
    hipLaunchKernelGGL(epilogue_kernel<8192>, dim3(1), dim3(XNT), 0, st, P);
}

int epilogue_work_vectors() { return N_WORK; }

}  // namespace kb
