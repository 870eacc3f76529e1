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
    const double dd = (norm >= TINY) ? -scale * exp2(Ev[s]) / ((double)S * norm) : 0.0;
    qE[s] = a_E[s] + qE[s] + dd;
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

void launch_epilogue(const EpiParams& P, hipStream_t st) {
  if (P.S <= 2048)
    hipLaunchKernelGGL(epilogue_kernel<2048>, dim3(1), dim3(XNT), 0, st, P);
  else
    hipLaunchKernelGGL(epilogue_kernel<8192>, dim3(1), dim3(XNT), 0, st, P);
}

int epilogue_work_vectors() { return N_WORK; }

}  // namespace kb
