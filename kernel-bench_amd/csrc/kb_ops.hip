// Per-wrapper kernels: the native launchers beneath the drop-in replacements
// of the reference's kbench/core/kernels/*.py wrappers (declarations and the
// reference function each replaces: include/kbench_ops.h).
//
// Design (MI355X):
//  * one 1024-thread workgroup per row (item row, clade row, split or split
//    side); thread t owns states t + k*1024 (k < CPT), so global row accesses
//    are coalesced;
//  * the species tree is described once by preorder positions and an Euler
//    tour (kb_tree); ancestors-or-self path sums are one prefix scan over the
//    Euler tour (+x on entry, -x on exit) and subtree sums one prefix scan
//    over preorder positions, both in LDS, independent of the tree depth;
//  * the E-step kernels (O(S) work) run in float64 and sum over tree levels;
//  * no atomics: cross-row accumulations are written as rows and summed in a
//    fixed order by kb_rows_scatter_add / kb_rows_sum_into.
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <type_traits>
#include <vector>

#include "kb_ops_common.hpp"

namespace kbo {

// ---- E-step -------------------------------------------------------------------

template <typename T>
struct EsArgs {
  int G, S, mode, use_col, max_iter;
  double tol;
  const T *E, *pS, *pD, *pL, *mt, *col;
  T *E_out, *Es1, *Es2, *Ebar, *max_diff;
  int* n_iter;
};

// One E-step of row values E (LDS, float64 log2) -> new values in En[k],
// plus E_s1, E_s2, Ebar in registers.  X is LDS scratch (S doubles).
template <typename T, int CPT>
__device__ void estep_eval(const OpsTree& t, const EsArgs<T>& a, size_t base, const double* Ev, double* X,
                           double* red, double (&En)[CPT], double (&Es1)[CPT], double (&Es2)[CPT],
                           double (&Eb)[CPT]) {
  const int S = t.S;
  const double NI = -__builtin_inf();
  double wE[CPT];
  double lm = NI;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    wE[k] = NI;
    if (s < S) {
      wE[k] = Ev[s] + (a.use_col ? (double)a.col[s] : 0.0);
      lm = fmax(lm, wE[k]);
    }
  }
  const double M = block_max(lm, red);
  const double Ms = M == NI ? 0.0 : M;
  double ls = 0.0;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      const double x = exp2(wE[k] - Ms);
      X[s] = x;
      ls += x;
    }
  }
  const double rowsum = block_sum(ls, red);  // its barrier publishes X
  level_path_sums(t, X);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      const size_t i = base + s;
      const int c1 = t.c1[s], c2 = t.c2[s];
      Es1[k] = c1 >= 0 ? Ev[c1] : NI;
      Es2[k] = c2 >= 0 ? Ev[c2] : NI;
      const double denom = rowsum - X[s];
      Eb[k] = denom > 0.0 ? log2(denom) + M + (double)a.mt[i] : NI;
      const double E = Ev[s];
      const double t0 = (double)a.pS[i] + Es1[k] + Es2[k];
      const double t1 = (double)a.pD[i] + 2.0 * E;
      const double t2 = E + Eb[k];
      const double t3 = (double)a.pL[i];
      const double m = fmax(fmax(t0, t1), fmax(t2, t3));
      const double ms = m == NI ? 0.0 : m;
      En[k] = log2(exp2(t0 - ms) + exp2(t1 - ms) + exp2(t2 - ms) + exp2(t3 - ms)) + m;
    }
  }
  __syncthreads();  // X and Ev reads done before the caller rewrites them
}

template <typename T, int CPT>
__global__ __launch_bounds__(NT) void estep_kernel(OpsTree t, EsArgs<T> a) {
  extern __shared__ double sm[];
  double* Ev = sm;
  double* X = sm + t.S;
  __shared__ double red[NW];
  const int S = t.S;
  const size_t base = (size_t)blockIdx.x * S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) Ev[s] = (double)a.E[base + s];
  }
  __syncthreads();
  double En[CPT], Es1[CPT], Es2[CPT], Eb[CPT];
  if (a.mode == 0) {
    estep_eval<T, CPT>(t, a, base, Ev, X, red, En, Es1, Es2, Eb);
    double ld = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) {
        const T en = (T)En[k];
        a.E_out[base + s] = en;
        a.Es1[base + s] = (T)Es1[k];
        a.Es2[base + s] = (T)Es2[k];
        a.Ebar[base + s] = (T)Eb[k];
        const T d = en - a.E[base + s];
        ld = fmax(ld, (double)(d < T(0) ? -d : d));
      }
    }
    const double md = block_max(ld, red);
    if (a.max_diff && threadIdx.x == 0) a.max_diff[blockIdx.x] = (T)md;
    return;
  }
  // fixed point: iterate while max |E_new - E| >= tol
  int it = 0;
  for (;;) {
    estep_eval<T, CPT>(t, a, base, Ev, X, red, En, Es1, Es2, Eb);
    double ld = 0.0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) {
        const double d = En[k] - Ev[s];
        if (!(fabs(d) < a.tol) && !(En[k] == Ev[s])) ld = fmax(ld, d != d ? __builtin_inf() : fabs(d));
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) Ev[s] = En[k];
    }
    ++it;
    const double md = block_max(ld, red);  // barrier also publishes Ev
    if (md < a.tol || it >= a.max_iter) break;
  }
  estep_eval<T, CPT>(t, a, base, Ev, X, red, En, Es1, Es2, Eb);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      a.E_out[base + s] = (T)Ev[s];
      a.Es1[base + s] = (T)Es1[k];
      a.Es2[base + s] = (T)Es2[k];
      a.Ebar[base + s] = (T)Eb[k];
    }
  }
  if (a.n_iter && threadIdx.x == 0) a.n_iter[blockIdx.x] = it;
}

template <typename T>
struct EvArgs {
  int G, S, use_col;
  const T *E, *En, *Es1, *Es2, *Ebar, *pS, *pD, *pL, *col, *gN, *g1, *g2, *gB;
  T *gE, *gpS, *gpD, *gpL, *gmt;
  double* work;  // [G, S] per-row contribution to grad_col
};

template <typename T, int CPT>
__global__ __launch_bounds__(NT) void estep_vjp_kernel(OpsTree t, EvArgs<T> a) {
  extern __shared__ double sm[];
  double* X = sm;       // r, then path sums, then u / subtree sums
  double* PC = sm + t.S;  // q0 + g_s1 / q0 + g_s2 of each column's parent
  __shared__ double red[NW];
  const int S = t.S;
  const size_t base = (size_t)blockIdx.x * S;
  const double NI = -__builtin_inf();
  double r[CPT], wbar[CPT], ge[CPT];
  double lm = NI;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    r[k] = NI;
    if (s < S) {
      r[k] = (double)a.E[base + s] + (a.use_col ? (double)a.col[s] : 0.0);
      lm = fmax(lm, r[k]);
      PC[s] = 0.0;
    }
  }
  const double M = block_max(lm, red);
  const double Ms = M == NI ? 0.0 : M;
  double ls = 0.0;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      r[k] = exp2(r[k] - Ms);
      X[s] = r[k];
      ls += r[k];
    }
  }
  const double rowsum = block_sum(ls, red);
  level_path_sums(t, X);
  double lu = 0.0;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    wbar[k] = 0.0;
    ge[k] = 0.0;
    if (s < S) {
      const size_t i = base + s;
      const double En = a.En[i], E = a.E[i];
      const double gN = a.gN[i];
      const double t0 = (double)a.pS[i] + (double)a.Es1[i] + (double)a.Es2[i];
      const double t1 = (double)a.pD[i] + 2.0 * E;
      const double t2 = E + (double)a.Ebar[i];
      const double t3 = (double)a.pL[i];
      const double q0 = gN * exp2(t0 - En), q1 = gN * exp2(t1 - En);
      const double q2 = gN * exp2(t2 - En), q3 = gN * exp2(t3 - En);
      wbar[k] = q2 + (double)a.gB[i];
      a.gpS[i] = (T)q0;
      a.gpD[i] = (T)q1;
      a.gpL[i] = (T)q3;
      a.gmt[i] = (T)wbar[k];
      ge[k] = 2.0 * q1 + q2;
      const int c1 = t.c1[s], c2 = t.c2[s];
      if (c1 >= 0) PC[c1] = q0 + (double)a.g1[i];
      if (c2 >= 0) PC[c2] = q0 + (double)a.g2[i];
      const double denom = rowsum - X[s];
      const double u = denom > 0.0 ? wbar[k] / denom : 0.0;
      lu += u;
      wbar[k] = u;  // reuse: u
    }
  }
  const double total_u = block_sum(lu, red);  // barrier: X reads and PC writes done
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) X[s] = wbar[k];
  }
  __syncthreads();
  level_subtree_sums(t, X);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      const double pv = r[k] * (total_u - X[s]);
      a.gE[base + s] = (T)(ge[k] + PC[s] + pv);
      a.work[base + s] = pv;
    }
  }
}

// ---- wave rows ------------------------------------------------------------------

template <typename T>
struct WsArgs {
  int S, W, use_col, use_leaf, store_final, n_sweeps;
  long long ws, pi_ws, cstride;
  const T* Pi_in;
  T *Pi_out, *Pibar, *rowmax;
  float* resid;
  const T *dts, *mt, *DL, *Ebar, *E, *SL1, *SL2, *col;
  const int64_t *item, *leaf_state;
  const T* leaf_logp;
};

// n_sweeps self-loop sweeps of one row; between sweeps the row stays in LDS
// (Pr), so the result equals n_sweeps one-sweep launches bit for bit.  The
// thread's tree entries (children, Euler events, entry events) and the row's
// constants are read once, before the first sweep.
template <typename T, int CPT>
__global__ __launch_bounds__(NT) void wave_step_kernel(OpsTree t, WsArgs<T> a) {
  extern __shared__ unsigned char smraw[];
  T* Pr = reinterpret_cast<T*>(smraw);  // input row, later the final-Pibar work row
  T* X = Pr + t.S;                      // linear row, then path sums, then the new row
  T* EV = X + t.S;                      // 2S Euler scan
  __shared__ T red[NW];
  const int S = t.S;
  const int w = blockIdx.x;
  const long long grow = a.ws + w;
  const T NI = ninf<T>();
  const long long item = a.item[grow];
  const size_t cb = (size_t)(item * a.cstride);
  const T* in = a.Pi_in + (size_t)(a.pi_ws + w) * S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) Pr[s] = in[s];
  }
  const long long lstate = a.use_leaf ? a.leaf_state[grow] : -1;
  int c1v[CPT], c2v[CPT], tinv[CPT], evv[2 * CPT];
  T kmt[CPT], kDL[CPT], kEb[CPT], kE[CPT], kS1[CPT], kS2[CPT], klf[CPT], kd[CPT], kcol[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    c1v[k] = c2v[k] = -1;
    tinv[k] = 0;
    kmt[k] = kDL[k] = kEb[k] = kE[k] = kS1[k] = kS2[k] = kcol[k] = T(0);
    klf[k] = kd[k] = NI;
    if (s < S) {
      const size_t ci = cb + s;
      c1v[k] = t.c1[s];
      c2v[k] = t.c2[s];
      tinv[k] = t.tin[s];
      kmt[k] = a.mt[ci];
      kDL[k] = a.DL[ci];
      kEb[k] = a.Ebar[ci];
      kE[k] = a.E[ci];
      kS1[k] = a.SL1[ci];
      kS2[k] = a.SL2[ci];
      if (lstate == s) klf[k] = a.leaf_logp[(size_t)item * S + s];
      if (a.dts) kd[k] = a.dts[(size_t)w * S + s];
      if (a.use_col) kcol[k] = a.col[s];
    }
  }
#pragma unroll
  for (int j = 0; j < 2 * CPT; ++j) {
    const int q = threadIdx.x + j * NT;
    evv[j] = q < 2 * S ? t.ev[q] : 0;
  }
  // ancestors-or-self path sums of x (LDS, column order) into ps (may alias x):
  // +x at the entry event and -x at the exit event of each column, scanned,
  // read back at the entry event
  auto path_sums_own = [&](const T* x, T* ps) {
#pragma unroll
    for (int j = 0; j < 2 * CPT; ++j) {
      const int q = threadIdx.x + j * NT;
      if (q < 2 * S) {
        const int e = evv[j];
        const T v = x[e >> 1];
        EV[q] = (e & 1) ? -v : v;
      }
    }
    __syncthreads();
    block_scan(EV, 2 * S, red);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) ps[s] = EV[tinv[k]];
    }
    __syncthreads();
  };
  __syncthreads();
  T wv[CPT], res[CPT];
  T ldiff = 0;
  for (int sweep = 0; sweep < a.n_sweeps; ++sweep) {
    // row max / sum of (col +) Pi, then Pibar(Pi) = log2(rowsum - pathsum) + M + mt
    T lm = NI;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      wv[k] = NI;
      if (s < S) {
        wv[k] = a.use_col ? kcol[k] + Pr[s] : Pr[s];
        lm = tmax(lm, wv[k]);
      }
    }
    const T M = block_max(lm, red);
    const T Ms = msafe(M);
    T ls = 0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) {
        const T x = xexp2(wv[k] - Ms);
        X[s] = x;
        ls += x;
      }
    }
    const T rowsum = block_sum(ls, red);
    path_sums_own(X, X);
    ldiff = 0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      res[k] = NI;
      if (s < S) {
        const T denom = rowsum - X[s];
        const T pibar_w = denom > T(0) ? xlog2(denom) + M + kmt[k] : NI;
        const T pi_w = Pr[s];
        const T ps1 = c1v[k] >= 0 ? Pr[c1v[k]] : NI;
        const T ps2 = c2v[k] >= 0 ? Pr[c2v[k]] : NI;
        const T t0 = kDL[k] + pi_w;
        const T t1 = pi_w + kEb[k];
        const T t2 = pibar_w + kE[k];
        const T t3 = kS1[k] + ps1;
        const T t4 = kS2[k] + ps2;
        const T t5 = klf[k];
        T m = tmax(tmax(tmax(t0, t1), tmax(t2, t3)), tmax(t4, t5));
        const T d = kd[k];
        if (a.dts) m = tmax(m, d);
        const T ms = msafe(m);
        T sum = xexp2(t0 - ms) + xexp2(t1 - ms) + xexp2(t2 - ms) + xexp2(t3 - ms) + xexp2(t4 - ms) + xexp2(t5 - ms);
        if (a.dts) sum += xexp2(d - ms);
        res[k] = xlog2(sum) + m;
        if (res[k] != NI && pi_w != NI) {
          const T df = res[k] - pi_w;
          ldiff = tmax(ldiff, df < T(0) ? -df : df);
        }
      }
    }
    __syncthreads();  // every read of X / Pr above is done
    if (sweep + 1 < a.n_sweeps) {
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int s = threadIdx.x + k * NT;
        if (s < S) Pr[s] = res[k];
      }
      __syncthreads();
    }
  }
  T* out = a.Pi_out + (size_t)grow * S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) out[s] = res[k];
  }
  if (a.resid) {
    const T md = block_max(ldiff, red);
    if (threadIdx.x == 0) a.resid[grow] = (float)md;
  }
  if (!a.store_final) return;
  __syncthreads();
  T lm2 = NI;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    wv[k] = NI;
    if (s < S) {
      wv[k] = a.use_col ? kcol[k] + res[k] : res[k];
      lm2 = tmax(lm2, wv[k]);
    }
  }
  const T M2 = block_max(lm2, red);
  const T Ms2 = msafe(M2);
  T ls2 = 0;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      const T x = xexp2(wv[k] - Ms2);
      Pr[s] = x;
      ls2 += x;
    }
  }
  const T rowsum2 = block_sum(ls2, red);
  path_sums_own(Pr, Pr);
  T* pb = a.Pibar + (size_t)grow * S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      const T denom = rowsum2 - Pr[s];
      pb[s] = denom > T(0) ? xlog2(denom) + M2 + kmt[k] : NI;
    }
  }
  if (threadIdx.x == 0) a.rowmax[grow] = M2;
}

// Sweep chains (n_sweeps > 1) of float32 rows in linear space, as the
// whole-pass forward row kernel runs its sweeps: x = 2^(Pi - M) with a row
// exponent M renormalised by an exact power of two every sweep, so a sweep is
//   y' = a y + emc (rowsum - ps) + k1 y[c1] + k2 y[c2] + (leaf | dts) 2^-M
// with a = 2^DL + 2^Ebar, emc = 2^(E + mt), k1 = 2^SL1, k2 = 2^SL2 formed
// once per launch, and no exponential or logarithm inside the chain.  The
// path sums come from an inclusive preorder scan and an exclusive postorder
// scan (two barriers per sweep).  The outputs equal the log-space sweeps to
// float32 rounding.
template <int CPT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(kb::pre_waves_per_eu(CPT)))) void wave_step_lin_kernel(OpsTree t, WsArgs<float> a) {
  constexpr int MAXS = NT * CPT;
  constexpr int LD = MAXS + 64;
  constexpr int ZERO = MAXS;     // padding slot: 0 in X
  constexpr int SEG = 64 * CPT;  // postorder slots per wavefront
  extern __shared__ __align__(16) unsigned char smraw[];
  float* X = reinterpret_cast<float*>(smraw);  // y of the sweep at preorder positions
  float* Q = X + LD;                           // exclusive postorder scan
  float* O = Q + LD;                           // the input row, then the outputs, at preorder positions
  __shared__ float wP[NW], wQ[NW], wM[NW];
  const int S = t.S;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int w = blockIdx.x;
  const long long grow = a.ws + w;
  const float NI = -__builtin_inff();
  const long long item = a.item[grow];
  const size_t cb = (size_t)(item * a.cstride);
  const float* in = a.Pi_in + (size_t)(a.pi_ws + w) * S;
  const long long lstate = a.use_leaf ? a.leaf_state[grow] : -1;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) O[t.ppos[sc]] = in[sc];
  }
  if (tid < 64) {
    X[MAXS + tid] = 0.0f;
    Q[MAXS + tid] = 0.0f;
  }
  // own positions: tables, the linear constants, and the log2 terms of the outputs
  int c1p[CPT], c2p[CPT], nex[CPT], qp[CPT];
  bool okp[CPT];
  float ca[CPT], ce[CPT], ck1[CPT], ck2[CPT], cw[CPT], cwq[CPT], kmt[CPT], kcol[CPT], klf[CPT], kd[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = kb::own_pos_c<NT, CPT>(k);
    okp[k] = i < S;
    c1p[k] = c2p[k] = ZERO;
    nex[k] = 0;
    qp[k] = ZERO;
    ca[k] = ce[k] = ck1[k] = ck2[k] = kmt[k] = kcol[k] = 0.0f;
    cw[k] = cwq[k] = a.use_col ? 0.0f : 1.0f;
    klf[k] = kd[k] = NI;
    if (okp[k]) {
      const int col = t.pcol[i];
      const size_t ci = cb + col;
      const int c1 = t.pc1[i], c2 = t.pc2[i];
      c1p[k] = c1 >= 0 ? c1 : ZERO;
      c2p[k] = c2 >= 0 ? c2 : ZERO;
      nex[k] = t.pnex[i];
      qp[k] = t.ppost[i];
      ca[k] = (float)(exp2((double)a.DL[ci]) + exp2((double)a.Ebar[ci]));
      ce[k] = (float)exp2((double)a.E[ci] + (double)a.mt[ci]);
      ck1[k] = c1 >= 0 ? (float)exp2((double)a.SL1[ci]) : 0.0f;
      ck2[k] = c2 >= 0 ? (float)exp2((double)a.SL2[ci]) : 0.0f;
      kmt[k] = a.mt[ci];
      if (a.use_col) {
        kcol[k] = a.col[col];
        cw[k] = exp2f(kcol[k]);
        cwq[k] = exp2f(a.col[t.pcol[qp[k]]]);
      }
      if (lstate == col) klf[k] = a.leaf_logp[(size_t)item * S + col];
      if (a.dts) kd[k] = a.dts[(size_t)w * S + col];
    }
  }
  __syncthreads();
  float pr[CPT];
  kb::lds_load_own<CPT>(O, pr);
  float lm = NI;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    if (!okp[k]) pr[k] = NI;
    lm = fmaxf(lm, pr[k]);
  }
  // linear space relative to the input's row maximum Ms
  const float Ms = kb::fsafe(kb::block_max1<NT>(lm, wM));
  float y[CPT], dl[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    y[k] = okp[k] ? exp2f(pr[k] - Ms) : 0.0f;
    dl[k] = (klf[k] != NI ? exp2f(klf[k] - Ms) : 0.0f) + (kd[k] != NI ? exp2f(kd[k] - Ms) : 0.0f);
  }
  int kexp = 0, kexp_prev = 0;
  float ps[CPT], yprev[CPT], rowsum = 0.0f, tsum = 0.0f, f = 1.0f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) yprev[k] = y[k];
  for (int sweep = 0;; ++sweep) {
    // phase A: publish y; inclusive (column-weighted) preorder scan in registers
    float sp[CPT], ta = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      ta += cw[k] * y[k];
      sp[k] = ta;
    }
    const float wa = kb::wave_scan_incl(ta);
    kb::lds_store_own<CPT>(X, y);
    if (lane == 63) wP[wv] = wa;
    __syncthreads();
    // phase B: row sum (renormalised by an exact power of two), the postorder
    // values and children (read before the next barrier), exclusive postorder scan
    const float tp = kb::lds_wave_values<NW>(wP, lane, 0.0f);
    float yq[CPT], x1[CPT], x2[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      yq[k] = X[qp[k]];
      x1[k] = X[c1p[k]];
      x2[k] = X[c2p[k]];
    }
    const float ip = kb::wave_scan_first<NW>(tp);
    tsum = kb::lane_value(ip, NW - 1);
    const float offp = kb::lane_value(ip - tp, wv) + (wa - ta);
    float sq[CPT], tb = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      sq[k] = tb;
      tb += cwq[k] * yq[k];
    }
    const float wb = kb::wave_scan_incl(tb);
#pragma unroll
    for (int k = 0; k < CPT; ++k) sq[k] += wb - tb;
    kb::lds_store_own<CPT>(Q, sq);
    if (lane == 63) wQ[wv] = wb;
    const int e = tsum > 0.0f ? __builtin_amdgcn_frexp_expf(tsum) : 0;
    f = __builtin_amdgcn_ldexpf(1.0f, -e);
    kexp += e;
    rowsum = tsum * f;
    __syncthreads();
    // phase C: path sums ps(i) = Pre(i) - PostEx(tin(i) - i)
    const float tq = kb::lds_wave_values<NW>(wQ, lane, 0.0f);
    const float eq = kb::wave_scan_first<NW>(tq) - tq;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int n = nex[k];
      ps[k] = (sp[k] + offp) - (Q[n] + __shfl(eq, n / SEG, 64));
    }
    if (sweep == a.n_sweeps) break;
    if (sweep == a.n_sweeps - 1) {  // the row before the last sweep, for the residual
#pragma unroll
      for (int k = 0; k < CPT; ++k) yprev[k] = y[k];
      kexp_prev = kexp - e;
    }
    const float scale = __builtin_amdgcn_ldexpf(1.0f, -kexp);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      float z = ca[k] * y[k];
      z += ck1[k] * x1[k];
      z += ck2[k] * x2[k];
      z += ce[k] * fmaxf(tsum - ps[k], 0.0f);
      y[k] = z * f + dl[k] * scale;
    }
  }
  // ---- outputs: Pi, the residual of the last sweep, Pibar and the row max
  const float M = Ms + (float)kexp;  // relative exponent of x = y f
  float po[CPT], pb[CPT];
  float ldiff = 0.0f, lmax = NI;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    po[k] = pb[k] = NI;
    if (okp[k]) {
      const float x = y[k] * f;
      po[k] = x > 0.0f ? log2f(x) + M : NI;
      const float prev = yprev[k] > 0.0f ? log2f(yprev[k]) + (Ms + (float)kexp_prev) : NI;
      if (po[k] != NI && prev != NI) ldiff = fmaxf(ldiff, fabsf(po[k] - prev));
      const float na = rowsum - ps[k] * f;
      pb[k] = na > 0.0f ? log2f(na) + M + kmt[k] : NI;
      lmax = fmaxf(lmax, kcol[k] + po[k]);
    }
  }
  // O (the input) was last read before the first sweep's barrier; X's readers
  // finished before the last pass's second barrier
  kb::lds_store_own<CPT>(O, po);
  kb::lds_store_own<CPT>(X, pb);
  __syncthreads();
  float* out = a.Pi_out + (size_t)grow * S;
  float* pbo = a.store_final ? a.Pibar + (size_t)grow * S : nullptr;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) {
      const int i = t.ppos[sc];
      out[sc] = O[i];
      if (pbo) pbo[sc] = X[i];
    }
  }
  if (a.resid) {
    const float md = kb::block_max1<NT>(ldiff, wM);
    if (tid == 0) a.resid[grow] = md;
  }
  if (a.store_final) {
    const float rmax = kb::block_max1<NT>(lmax, wP);
    if (tid == 0) a.rowmax[grow] = rmax;
  }
}

template <typename T>
struct LiArgs {
  int S, W, use_col;
  long long ws, cstride;
  T* Pi_out;
  const T *mt, *DL, *Ebar, *E, *SL1, *SL2, *col;
  const int64_t *sub_start, *sub_end, *item, *leaf_state, *c1, *c2;
  const T* leaf_logp;
};

template <typename T>
__global__ __launch_bounds__(256) void leaf_init_kernel(LiArgs<T> a) {
  const int w = blockIdx.x;
  const int s = blockIdx.y * 256 + threadIdx.x;
  const int S = a.S;
  if (s >= S) return;
  const T NI = ninf<T>();
  const long long grow = a.ws + w;
  const long long item = a.item[grow];
  const size_t ci = (size_t)(item * a.cstride) + s;
  const long long leaf = a.leaf_state[grow];
  const bool valid_leaf = leaf >= 0 && leaf < S;
  const long long ls = valid_leaf ? a.sub_start[leaf] : 0, le = valid_leaf ? a.sub_end[leaf] : 0;
  const long long st = a.sub_start[s];
  const bool desc = valid_leaf && st >= ls && st < le;
  const bool hit = s == leaf;
  const T lcol = (a.use_col && valid_leaf) ? a.col[leaf] : T(0);
  const T obs = valid_leaf ? a.leaf_logp[(size_t)item * S + leaf] : NI;
  const T pi_w = hit ? obs : NI;
  const T pibar_w = desc ? NI : a.mt[ci] + lcol + obs;
  const int c1 = child_at(a.c1, s, S), c2 = child_at(a.c2, s, S);
  const T ps1 = (c1 >= 0 && c1 == leaf) ? obs : NI;
  const T ps2 = (c2 >= 0 && c2 == leaf) ? obs : NI;
  const T t0 = a.DL[ci] + pi_w;
  const T t1 = pi_w + a.Ebar[ci];
  const T t2 = pibar_w + a.E[ci];
  const T t3 = a.SL1[ci] + ps1;
  const T t4 = a.SL2[ci] + ps2;
  const T t5 = hit ? a.leaf_logp[(size_t)item * S + s] : NI;
  const T m = tmax(tmax(tmax(t0, t1), tmax(t2, t3)), tmax(t4, t5));
  const T ms = msafe(m);
  const T sum = xexp2(t0 - ms) + xexp2(t1 - ms) + xexp2(t2 - ms) + xexp2(t3 - ms) + xexp2(t4 - ms) + xexp2(t5 - ms);
  a.Pi_out[(size_t)grow * S + s] = xlog2(sum) + m;
}

// ---- split reduction --------------------------------------------------------------

template <typename T>
struct DtsArgs {
  int S, W, by_state;
  long long item_offset, prow;
  const T *Pi, *Pibar, *lsp, *pD, *pS;
  const int64_t *sl, *sr, *item, *c1, *c2;
  const int *ptr, *order;
  const uint8_t* active;
  T* out;
};

template <typename T, int CPT>
__global__ __launch_bounds__(NT) void dts_kernel(DtsArgs<T> a) {
  const int S = a.S;
  const int w = blockIdx.x;
  const T NI = ninf<T>();
  T* out = a.out + (size_t)w * S;
  const int b = a.ptr[w], e = a.ptr[w + 1];
  if ((a.active && !a.active[w]) || b == e) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) out[s] = NI;
    }
    return;
  }
  const long long item = a.item[a.item_offset + w];
  const size_t pb = (size_t)(item * a.prow);
  T m[CPT], acc[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    m[k] = NI;
    acc[k] = 0;
  }
  for (int j = b; j < e; ++j) {
    const int si = a.order[j];
    const T* Pl = a.Pi + (size_t)a.sl[si] * S;
    const T* Pr = a.Pi + (size_t)a.sr[si] * S;
    const T* Bl = a.Pibar + (size_t)a.sl[si] * S;
    const T* Br = a.Pibar + (size_t)a.sr[si] * S;
    const T lsp = a.lsp[si];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) {
        const T d = a.by_state ? a.pD[pb + s] : a.pD[pb];
        const T sp = a.by_state ? a.pS[pb + s] : a.pS[pb];
        const T pl = Pl[s], pr = Pr[s];
        const int c1 = child_at(a.c1, s, S), c2 = child_at(a.c2, s, S);
        const T l1 = c1 >= 0 ? Pl[c1] : NI, r1 = c1 >= 0 ? Pr[c1] : NI;
        const T l2 = c2 >= 0 ? Pl[c2] : NI, r2 = c2 >= 0 ? Pr[c2] : NI;
        const T v0 = lsp + d + pl + pr;
        const T v1 = lsp + pl + Br[s];
        const T v2 = lsp + pr + Bl[s];
        const T v3 = lsp + sp + l1 + r2;
        const T v4 = lsp + sp + r1 + l2;
        const T sm = tmax(tmax(tmax(v0, v1), tmax(v2, v3)), v4);
        const T sms = msafe(sm);
        const T ss = xexp2(v0 - sms) + xexp2(v1 - sms) + xexp2(v2 - sms) + xexp2(v3 - sms) + xexp2(v4 - sms);
        const T nm = tmax(m[k], sm);
        const T nms = msafe(nm);
        acc[k] = (m[k] != NI ? acc[k] * xexp2(m[k] - nms) : T(0)) + ss * xexp2(sms - nms);
        m[k] = nm;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) out[s] = xlog2(acc[k]) + m[k];
  }
}

// ---- active mask ------------------------------------------------------------------------

__device__ __forceinline__ float absval(float x) { return fabsf(x); }
__device__ __forceinline__ double absval(double x) { return fabs(x); }

template <typename T>
__device__ __forceinline__ double as_double(T x) {
  return (double)x;
}
template <>
__device__ __forceinline__ double as_double<__hip_bfloat16>(__hip_bfloat16 x) {
  return (double)__bfloat162float(x);
}

template <typename T>
__global__ __launch_bounds__(256) void active_kernel(int S, long long stride, const T* rhs, float thr, int strict,
                                                     uint8_t* active) {
  __shared__ double red[4];
  const T* row = rhs + (size_t)blockIdx.x * stride;
  double m = 0.0;
  for (int s = threadIdx.x; s < S; s += 256) {
    const double v = fabs(as_double(row[s]));
    m = v > m || v != v ? v : m;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const double y = __shfl_xor(m, o, 64);
    m = y > m || y != y ? y : m;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    double r = red[0];
    for (int i = 1; i < 4; ++i) r = red[i] > r || red[i] != red[i] ? red[i] : r;
    // compare in the row's precision against the float32 threshold, as a
    // Triton kernel does with a Python float argument
    const double th = (double)thr;
    active[blockIdx.x] = strict ? (r > th) : (r >= th);
  }
}

// ---- self-loop adjoint ---------------------------------------------------------------------

template <typename T>
struct WbArgs {
  int S, W, n_terms, clayout, leaf_mode, use_leaf, use_col;
  long long ws;
  const T *Pi, *Pibar, *rowmax, *dts, *rhs, *v0;
  const uint8_t* active;
  const T *mt, *DL, *Ebar, *E, *SL1, *SL2, *col;
  const int64_t *item, *leaf_state;
  const T *leaf_logp, *leaf_term;
  T *v, *aw0, *aw1, *aw2, *aw345, *aw3, *aw4, *col_rows;
  float* relres;
};

template <typename T, int CPT>
__global__ __launch_bounds__(NT) void wave_bwd_kernel(OpsTree t, WbArgs<T> a) {
  extern __shared__ unsigned char smraw[];
  T* X = reinterpret_cast<T*>(smraw);  // p', then path sums
  T* Ed = X + t.S;                     // edge weight into each column from its parent
  T* Tm = Ed + t.S;                    // current Neumann term (column order)
  T* Up = Tm + t.S;                    // preorder scan of u; Tm..Up double as the 2S Euler scan
  __shared__ T red[NW];
  const int S = a.S;
  const int w = blockIdx.x;
  const long long grow = a.ws + w;
  const size_t ob = (size_t)w * S;
  const T NI = ninf<T>();
  const bool act = a.active ? a.active[w] != 0 : true;
  if (!act) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) {
        a.v[ob + s] = 0;
        a.aw0[ob + s] = 0;
        a.aw1[ob + s] = 0;
        a.aw2[ob + s] = 0;
        a.aw345[ob + s] = 0;
        a.aw3[ob + s] = 0;
        a.aw4[ob + s] = 0;
        a.col_rows[ob + s] = 0;
      }
    }
    if (a.relres && threadIdx.x == 0) a.relres[w] = 0.0f;
    return;
  }
  const long long item = a.item ? a.item[grow] : 0;
  const size_t cb = a.clayout == 1 ? ob : (a.clayout == 2 ? (size_t)item * S : 0);
  const T* pirow = a.Pi + (size_t)grow * S;
  const T* pbrow = a.Pibar + (size_t)grow * S;
  const T rms = msafe(a.rowmax[grow]);
  // p' and its row sum
  T pp[CPT];
  T ls = 0;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    pp[k] = 0;
    if (s < S) {
      pp[k] = xexp2((a.use_col ? a.col[s] + pirow[s] : pirow[s]) - rms);
      X[s] = pp[k];
      Ed[s] = 0;
      ls += pp[k];
    }
  }
  const T row_sum = block_sum(ls, red);
  path_sums(t, X, Tm, X, red);
  const long long lstate = a.use_leaf ? a.leaf_state[grow] : -1;
  T diag[CPT], pcoef[CPT], wl[CPT], e0[CPT], e1[CPT], e2[CPT], e3[CPT], e4[CPT], e5[CPT], isum[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    diag[k] = pcoef[k] = wl[k] = 0;
    e0[k] = e1[k] = e2[k] = e3[k] = e4[k] = e5[k] = isum[k] = 0;
    if (s < S) {
      const size_t ci = cb + s;
      const T pi = pirow[s];
      const int c1 = t.c1[s], c2 = t.c2[s];
      const T ps1 = c1 >= 0 ? pirow[c1] : NI;
      const T ps2 = c2 >= 0 ? pirow[c2] : NI;
      const T t0 = a.DL[ci] + pi;
      const T t1 = pi + a.Ebar[ci];
      const T t2 = pbrow[s] + a.E[ci];
      const T t3 = a.SL1[ci] + ps1;
      const T t4 = a.SL2[ci] + ps2;
      T t5 = NI;
      if (a.use_leaf) {
        if (lstate == s) {
          if (a.leaf_mode == 3) t5 = a.leaf_logp[0];
          else if (a.leaf_mode == 1) t5 = a.leaf_logp[item];
          else if (a.leaf_mode == 2) t5 = a.leaf_logp[(size_t)item * S + s];
          else t5 = a.leaf_logp[s];
        }
      } else if (a.leaf_term) {
        t5 = a.leaf_term[ob + s];
      }
      const T m = tmax(tmax(tmax(t0, t1), tmax(t2, t3)), tmax(t4, t5));
      const T ms = msafe(m);
      e0[k] = xexp2(t0 - ms);
      e1[k] = xexp2(t1 - ms);
      e2[k] = xexp2(t2 - ms);
      e3[k] = xexp2(t3 - ms);
      e4[k] = xexp2(t4 - ms);
      e5[k] = xexp2(t5 - ms);
      const T sum = e0[k] + e1[k] + e2[k] + e3[k] + e4[k] + e5[k];
      isum[k] = sum > T(0) ? T(1) / sum : T(0);
      wl[k] = 1;
      if (a.dts) {
        const T dl = xlog2(sum) + m;
        const T dr = a.dts[ob + s];
        const T pm = tmax(dl, dr);
        const T pms = msafe(pm);
        const T pnew = xlog2(xexp2(dl - pms) + xexp2(dr - pms)) + pm;
        wl[k] = dl != NI ? xexp2(dl - pnew) : T(0);
      }
      const T denom = row_sum - X[s];
      const T idn = denom > T(0) ? T(1) / denom : T(0);
      diag[k] = wl[k] * (e0[k] + e1[k]) * isum[k];
      pcoef[k] = wl[k] * e2[k] * isum[k] * idn;
      if (c1 >= 0) Ed[c1] = wl[k] * e3[k] * isum[k];
      if (c2 >= 0) Ed[c2] = wl[k] * e4[k] * isum[k];
    }
  }
  __syncthreads();
  T edge[CPT], term[CPT], v[CPT], rh[CPT];
  int par[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    edge[k] = s < S ? Ed[s] : T(0);
    par[k] = s < S ? t.par[s] : -1;
    rh[k] = s < S ? a.rhs[ob + s] : T(0);
    // Neumann: term_0 = rhs; fixed point from initial_v: the term is v itself
    v[k] = a.v0 ? (s < S ? a.v0[ob + s] : T(0)) : rh[k];
    term[k] = v[k];
  }
  // Neumann series v = sum_{n <= N} (J^T)^n rhs, or N steps of v <- rhs + J^T v
  for (int n = 0; n < a.n_terms; ++n) {
    T lu = 0;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) {
        Tm[s] = term[k];
        const T u = term[k] * pcoef[k];
        X[s] = u;
        lu += u;
      }
    }
    __syncthreads();
    subtree_scan(t, X, Up, red);
    const T A = Up[S - 1];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) {
        const T nt = term[k] * diag[k] + pp[k] * complement_of(t, Up, s, A) + (par[k] >= 0 ? Tm[par[k]] : T(0)) * edge[k];
        if (a.v0) {
          v[k] = rh[k] + nt;
          term[k] = v[k];
        } else {
          term[k] = nt;
          v[k] += nt;
        }
      }
    }
    __syncthreads();
  }
  // column gradient p' (A - subtree(v pcoef)) and the parameter contributions
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) X[s] = v[k] * pcoef[k];
  }
  __syncthreads();
  subtree_scan(t, X, Up, red);
  const T A = Up[S - 1];
  T ln = 0, lv = 0;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      a.col_rows[ob + s] = pp[k] * complement_of(t, Up, s, A);
      const T al = v[k] * wl[k] * isum[k];
      const T a3 = al * e3[k], a4 = al * e4[k], a5 = al * e5[k];
      a.v[ob + s] = v[k];
      a.aw0[ob + s] = al * e0[k];
      a.aw1[ob + s] = al * e1[k];
      a.aw2[ob + s] = al * e2[k];
      a.aw3[ob + s] = a3;
      a.aw4[ob + s] = a4;
      a.aw345[ob + s] = a3 + a4 + a5;
      const float tf = (float)term[k], vf = (float)v[k];
      ln += (T)(tf * tf);
      lv += (T)(vf * vf);
    }
  }
  if (a.relres) {
    const T n2 = block_sum(ln, red);
    const T v2 = block_sum(lv, red);
    if (threadIdx.x == 0) {
      const float tiny = 1.17549435e-38f;
      const float den = fmaxf(sqrtf((float)v2), tiny);
      a.relres[w] = a.n_terms > 0 ? sqrtf((float)n2) / den : 0.0f;
    }
  }
}

// float32 rows at preorder ownership (thread t owns positions t*CPT + k, as
// the whole-pass backward row kernel): the root-path sums of p' from an
// inclusive preorder and an exclusive postorder scan, one barrier per Neumann
// term (wavefront-local scans published, the readers add the wavefront
// offsets), and the [W, S] outputs written back in column order through LDS.
// Same mathematics as wave_bwd_kernel.
template <int CPT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(kb::pre_waves_per_eu(CPT)))) void wave_bwd_pre_kernel(OpsTree t, WbArgs<float> a) {
  constexpr int MAXS = NT * CPT;
  constexpr int LD = MAXS + 64;  // [MAXS] is the padding slot, kept at 0
  constexpr int ZERO = MAXS;
  constexpr int SEG = 64 * CPT;  // postorder slots per wavefront
  extern __shared__ __align__(16) unsigned char smraw[];
  float* L0 = reinterpret_cast<float*>(smraw);
  float* L1 = L0 + LD;
  float* L2 = L1 + LD;
  float* L3 = L2 + LD;
  __shared__ float wA[NW], wB[NW];
  const int S = a.S;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int w = blockIdx.x;
  const long long grow = a.ws + w;
  const size_t ob = (size_t)w * S;
  const float NI = -__builtin_inff();
  const bool act = a.active ? a.active[w] != 0 : true;
  if (!act) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      if (s < S) {
        a.v[ob + s] = 0;
        a.aw0[ob + s] = 0;
        a.aw1[ob + s] = 0;
        a.aw2[ob + s] = 0;
        a.aw345[ob + s] = 0;
        a.aw3[ob + s] = 0;
        a.aw4[ob + s] = 0;
        a.col_rows[ob + s] = 0;
      }
    }
    if (a.relres && tid == 0) a.relres[w] = 0.0f;
    return;
  }
  const long long item = a.item ? a.item[grow] : 0;
  const size_t cb = a.clayout == 1 ? ob : (a.clayout == 2 ? (size_t)item * S : 0);
  const float* pirow = a.Pi + (size_t)grow * S;
  const float* pbrow = a.Pibar + (size_t)grow * S;
  const float rms = msafe(a.rowmax[grow]);
  // Pi and Pibar to their preorder positions (coalesced column reads)
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) {
      const int p = t.ppos[sc];
      L0[p] = pirow[sc];
      L1[p] = pbrow[sc];
    }
  }
  if (tid < 64) {
    L0[MAXS + tid] = 0.0f;
    L1[MAXS + tid] = 0.0f;
    L2[MAXS + tid] = 0.0f;
    L3[MAXS + tid] = 0.0f;
  }
  // own positions: column, children, parent, subtree end - 1, postorder slot, tin - i
  int colk[CPT], c1p[CPT], c2p[CPT], ppar[CPT], endm1[CPT], wend[CPT], qp[CPT], nex[CPT];
  bool okp[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = kb::own_pos_c<NT, CPT>(k);
    okp[k] = i < S;
    colk[k] = okp[k] ? t.pcol[i] : 0;
    c1p[k] = okp[k] ? t.pc1[i] : -1;
    c2p[k] = okp[k] ? t.pc2[i] : -1;
    const int par = okp[k] ? t.par[colk[k]] : -1;
    ppar[k] = par >= 0 ? t.ppos[par] : ZERO;
    endm1[k] = okp[k] ? t.pend[colk[k]] - 1 : ZERO;
    wend[k] = endm1[k] < ZERO ? endm1[k] / SEG : 0;
    qp[k] = okp[k] ? t.ppost[i] : ZERO;
    nex[k] = okp[k] ? t.pnex[i] : 0;
  }
  __syncthreads();
  float piv[CPT], pbv[CPT];
  kb::lds_load_own<CPT>(L0, piv);
  kb::lds_load_own<CPT>(L1, pbv);
  // p' = 2^(col + Pi - rowmax) and its root-path sums ps(i) = Pre(i) - PostEx(tin(i) - i)
  float pp[CPT], sp[CPT], ta = 0.0f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    pp[k] = okp[k] ? xexp2((a.use_col ? a.col[colk[k]] + piv[k] : piv[k]) - rms) : 0.0f;
    ta += pp[k];
    sp[k] = ta;
  }
  const float wa = kb::wave_scan_incl(ta);
  kb::lds_store_own<CPT>(L2, pp);
  if (lane == 63) wA[wv] = wa;
  __syncthreads();
  float ps[CPT], ch1[CPT], ch2[CPT], row_sum;
  {
    const float tp = kb::lds_wave_values<NW>(wA, lane, 0.0f);
    float yq[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      yq[k] = L2[qp[k]];
      ch1[k] = c1p[k] >= 0 ? L0[c1p[k]] : NI;
      ch2[k] = c2p[k] >= 0 ? L0[c2p[k]] : NI;
    }
    const float ip = kb::wave_scan_first<NW>(tp);
    row_sum = kb::lane_value(ip, NW - 1);
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
    kb::lds_store_own<CPT>(L3, sq);
    if (lane == 63) wB[wv] = wb;
    __syncthreads();
    const float tq = kb::lds_wave_values<NW>(wB, lane, 0.0f);
    const float eq = kb::wave_scan_first<NW>(tq) - tq;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int n = nex[k];
      ps[k] = (sp[k] + offp) - (L3[n] + __shfl(eq, n / SEG, 64));
    }
  }
  // J^T coefficients; the child-edge weights (q3 into child1, q4 into child2)
  // scattered by the parent's owner into L1; the rhs and initial rows staged
  // into L2 / L0 (free since the scans above), all under one barrier
  const long long lstate = a.use_leaf ? a.leaf_state[grow] : -1;
  float diag[CPT], pcoef[CPT], q[6][CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    diag[k] = pcoef[k] = 0.0f;
#pragma unroll
    for (int j = 0; j < 6; ++j) q[j][k] = 0.0f;
    if (okp[k]) {
      const int s = colk[k];
      const size_t ci = cb + s;
      const float pi = piv[k];
      const float t0 = a.DL[ci] + pi;
      const float t1 = pi + a.Ebar[ci];
      const float t2 = pbv[k] + a.E[ci];
      const float t3 = a.SL1[ci] + ch1[k];
      const float t4 = a.SL2[ci] + ch2[k];
      float t5 = NI;
      if (a.use_leaf) {
        if (lstate == s) {
          if (a.leaf_mode == 3) t5 = a.leaf_logp[0];
          else if (a.leaf_mode == 1) t5 = a.leaf_logp[item];
          else if (a.leaf_mode == 2) t5 = a.leaf_logp[(size_t)item * S + s];
          else t5 = a.leaf_logp[s];
        }
      } else if (a.leaf_term) {
        t5 = a.leaf_term[ob + s];
      }
      const float m = tmax(tmax(tmax(t0, t1), tmax(t2, t3)), tmax(t4, t5));
      const float ms = msafe(m);
      const float e0 = xexp2(t0 - ms), e1 = xexp2(t1 - ms), e2 = xexp2(t2 - ms);
      const float e3 = xexp2(t3 - ms), e4 = xexp2(t4 - ms), e5 = xexp2(t5 - ms);
      const float sum = e0 + e1 + e2 + e3 + e4 + e5;
      const float isum = sum > 0.0f ? 1.0f / sum : 0.0f;
      float wl = 1.0f;
      if (a.dts) {
        const float dl = xlog2(sum) + m;
        const float dr = a.dts[ob + s];
        const float pm = tmax(dl, dr);
        const float pms = msafe(pm);
        const float pnew = xlog2(xexp2(dl - pms) + xexp2(dr - pms)) + pm;
        wl = dl != NI ? xexp2(dl - pnew) : 0.0f;
      }
      const float denom = row_sum - ps[k];
      const float idn = denom > 0.0f ? 1.0f / denom : 0.0f;
      diag[k] = wl * (e0 + e1) * isum;
      pcoef[k] = wl * e2 * isum * idn;
      const float c = wl * isum;
      q[0][k] = c * e0;
      q[1][k] = c * e1;
      q[2][k] = c * e2;
      q[3][k] = c * e3;
      q[4][k] = c * e4;
      q[5][k] = c * e5;
      if (c1p[k] >= 0) L1[c1p[k]] = wl * e3 * isum;
      if (c2p[k] >= 0) L1[c2p[k]] = wl * e4 * isum;
    }
  }
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) {
      const int p = t.ppos[sc];
      L2[p] = a.rhs[ob + sc];
      if (a.v0) L0[p] = a.v0[ob + sc];
    }
  }
  __syncthreads();
  float edge[CPT], rh[CPT], v[CPT], term[CPT];
  kb::lds_load_own<CPT>(L1, edge);
  kb::lds_load_own<CPT>(L2, rh);
  if (a.v0) kb::lds_load_own<CPT>(L0, v);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    edge[k] = ppar[k] != ZERO ? edge[k] : 0.0f;
    if (!okp[k]) rh[k] = 0.0f;
    // Neumann: term_0 = rhs; fixed point from initial_v: the term is v itself
    v[k] = a.v0 ? (okp[k] ? v[k] : 0.0f) : rh[k];
    term[k] = v[k];
  }
  // Neumann series v = sum_{n <= N} (J^T)^n rhs, or N steps of v <- rhs + J^T v.
  // Buffers alternate by parity: (Tb, Lb) = (L0, L2) for even terms, (L1, L3)
  // for odd ones; every thread read its own L0..L2 entries above, and the
  // other threads' entries are read only after each term's barrier.
  auto neumann_term = [&](float* Tb, float* Lb, float* wt) {
    float sc[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) sc[k] = term[k] * pcoef[k] + (k > 0 ? sc[k - 1] : 0.0f);
    const float tsum = sc[CPT - 1];
    const float ws = kb::wave_scan_incl(tsum);
    if (lane == 63) wt[wv] = ws;
#pragma unroll
    for (int k = 0; k < CPT; ++k) sc[k] += ws - tsum;
    kb::lds_store_own<CPT>(Lb, sc);
    kb::lds_store_own<CPT>(Tb, term);
    __syncthreads();
    float le[CPT], tpar[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      le[k] = Lb[endm1[k]];
      tpar[k] = Tb[ppar[k]];
    }
    const float wtot = lane < NW ? wt[lane] : 0.0f;
    const float wincl = kb::wave_scan_first<NW>(wtot);
    const float wexcl = wincl - wtot;
    const float A = kb::lane_value(wincl, NW - 1);
    const float woff = kb::lane_value(wexcl, wv);
    const float p0 = kb::wave_prev_lane(sc[CPT - 1]) + woff;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const float pm1 = k == 0 ? p0 : sc[k - 1] + woff;
      const float nt = term[k] * diag[k] + pp[k] * (pm1 + (A - (le[k] + __shfl(wexcl, wend[k], 64)))) +
                       tpar[k] * edge[k];
      if (a.v0) {
        v[k] = rh[k] + nt;
        term[k] = v[k];
      } else {
        term[k] = nt;
        v[k] += nt;
      }
    }
  };
  {
    int n = 0;
    for (; n + 2 <= a.n_terms; n += 2) {
      neumann_term(L0, L2, wA);
      neumann_term(L1, L3, wB);
    }
    if (n < a.n_terms) neumann_term(L0, L2, wA);
  }
  // column gradient p' (A - subtree(v pcoef)), in the next parity's buffers
  float colg[CPT];
  {
    const int n = a.n_terms;
    float* Pb = (n & 1) ? L3 : L2;
    float* wt = (n & 1) ? wB : wA;
    float u[CPT], sc[CPT], pm1[CPT], rest[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) u[k] = v[k] * pcoef[k];
    kb::local_scan_publish<NT, CPT>(sc, u, Pb, wt);
    __syncthreads();
    kb::subtree_terms<NT, CPT>(sc, Pb, wt, endm1, wend, pm1, rest);
#pragma unroll
    for (int k = 0; k < CPT; ++k) colg[k] = okp[k] ? pp[k] * (pm1[k] + rest[k]) : 0.0f;
  }
  // outputs in column order, four rows at a time through L0..L3
  float* const outs[8] = {a.v, a.aw0, a.aw1, a.aw2, a.aw3, a.aw4, a.aw345, a.col_rows};
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    __syncthreads();  // the previous readers of L0..L3 are done
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = 4 * half + r;
      float x[CPT];
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        if (o == 0) x[k] = v[k];
        else if (o == 7) x[k] = colg[k];
        else if (o == 6) x[k] = v[k] * (q[3][k] + q[4][k] + q[5][k]);
        else x[k] = v[k] * q[o - 1][k];
      }
      kb::lds_store_own<CPT>(L0 + r * LD, x);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* dst = outs[4 * half + r] + ob;
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        const int sc = tid + j * NT;
        if (sc < S) dst[sc] = L0[r * LD + t.ppos[sc]];
      }
    }
  }
  if (a.relres) {
    float ln = 0.0f, lv = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      ln += term[k] * term[k];
      lv += v[k] * v[k];
    }
    const float n2 = block_sum(ln, wA);
    const float v2 = block_sum(lv, wB);
    if (tid == 0) {
      const float tiny = 1.17549435e-38f;
      const float den = fmaxf(sqrtf(v2), tiny);
      a.relres[w] = a.n_terms > 0 ? sqrtf(n2) / den : 0.0f;
    }
  }
}

// ---- cross-wave split adjoint ----------------------------------------------------------------

template <typename T>
struct DcArgs {
  int S, playout, mlayout, output_ud, skip_zero;
  long long N, ws;
  double side_thr;
  const T *Pi, *Pibar, *v;
  const uint8_t* active;
  const int64_t *sl, *sr, *red_idx, *item, *c1, *c2;
  const T *wlsp, *pD, *pS, *mt, *rowmax;
  T *side_rows, *ud, *A;
  uint8_t* side_active;
  T *gPl, *gPr, *prow, *psum, *mrow;
};

template <typename T, int CPT>
__global__ __launch_bounds__(NT)
__attribute__((amdgpu_waves_per_eu(sizeof(T) == 4 ? kb::pre_waves_per_eu(CPT) : 1))) void dts_cross_kernel(DcArgs<T> a) {
  extern __shared__ unsigned char smraw[];
  T* Lr = reinterpret_cast<T*>(smraw);
  T* Rr = Lr + a.S;
  __shared__ T red[NW];
  const int S = a.S;
  const long long i = blockIdx.x;
  const long long N = a.N;
  const T NI = ninf<T>();
  const long long pw = a.red_idx[i];
  const bool act = a.active ? a.active[pw] != 0 : true;
  T* sideL = a.side_rows + (size_t)i * S;
  T* sideR = a.side_rows + (size_t)(N + i) * S;
  if (!act) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) {
        sideL[s] = 0;
        sideR[s] = 0;
        if (a.prow) {
          a.prow[(size_t)i * S + s] = 0;
          a.prow[(size_t)(N + i) * S + s] = 0;
        }
        if (a.mrow) {
          a.mrow[(size_t)i * S + s] = 0;
          a.mrow[(size_t)(N + i) * S + s] = 0;
        }
        if (a.output_ud) {
          if (!a.skip_zero) {
            a.ud[(size_t)i * S + s] = 0;
            a.ud[(size_t)(N + i) * S + s] = 0;
          }
        } else {
          a.gPl[(size_t)i * S + s] = 0;
          a.gPr[(size_t)i * S + s] = 0;
        }
      }
    }
    if (threadIdx.x == 0) {
      if (a.psum) {
        a.psum[i] = 0;
        a.psum[N + i] = 0;
      }
      if (a.output_ud) {
        if (a.side_active) {
          a.side_active[i] = 0;
          a.side_active[N + i] = 0;
        }
        if (!a.skip_zero) {
          a.A[i] = 0;
          a.A[N + i] = 0;
        }
      }
    }
    return;
  }
  const long long l = a.sl[i], r = a.sr[i];
  const long long prow_g = a.ws + pw;
  const long long pitem = a.item ? a.item[prow_g] : 0;
  const long long il = (a.item && a.mlayout == 1) ? a.item[l] : 0;
  const long long ir = (a.item && a.mlayout == 1) ? a.item[r] : 0;
  const T wlsp = a.wlsp[i];
  const T* Pl = a.Pi + (size_t)l * S;
  const T* Prr = a.Pi + (size_t)r * S;
  const T* Bl = a.Pibar + (size_t)l * S;
  const T* Br = a.Pibar + (size_t)r * S;
  const T* Pp = a.Pi + (size_t)prow_g * S;
  const T* vr = a.v + (size_t)pw * S;
  T vd3[CPT], vd4[CPT];
  int c1v[CPT], c2v[CPT];
  T sd = 0, ss = 0, sul = 0, sur = 0, bl = 0, br = 0;
  T rml = 0, rmr = 0;
  if (a.output_ud) {
    rml = a.rowmax[l];
    rmr = a.rowmax[r];
  }
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    vd3[k] = vd4[k] = 0;
    c1v[k] = c2v[k] = -1;
    if (s < S) {
      T d, sp;
      if (a.playout == 0) {
        d = a.pD[0];
        sp = a.pS[0];
      } else if (a.playout == 1) {
        d = a.pD[s];
        sp = a.pS[s];
      } else if (a.playout == 2) {
        d = a.pD[pitem];
        sp = a.pS[pitem];
      } else {
        d = a.pD[(size_t)pitem * S + s];
        sp = a.pS[(size_t)pitem * S + s];
      }
      const T pil = Pl[s], pir = Prr[s];
      const int c1 = child_at(a.c1, s, S), c2 = child_at(a.c2, s, S);
      c1v[k] = c1;
      c2v[k] = c2;
      const T l1 = c1 >= 0 ? Pl[c1] : NI, r1 = c1 >= 0 ? Prr[c1] : NI;
      const T l2 = c2 >= 0 ? Pl[c2] : NI, r2 = c2 >= 0 ? Prr[c2] : NI;
      const T d0 = d + pil + pir;
      const T d1 = pil + Br[s];
      const T d2 = pir + Bl[s];
      const T d3 = sp + l1 + r2;
      const T d4 = sp + r1 + l2;
      const T pp = Pp[s];
      const bool pv = pp != NI;
      const T vv = vr[s];
      const T vd0 = pv ? vv * xexp2(wlsp + d0 - pp) : T(0);
      const T vd1 = pv ? vv * xexp2(wlsp + d1 - pp) : T(0);
      const T vd2 = pv ? vv * xexp2(wlsp + d2 - pp) : T(0);
      vd3[k] = pv ? vv * xexp2(wlsp + d3 - pp) : T(0);
      vd4[k] = pv ? vv * xexp2(wlsp + d4 - pp) : T(0);
      Lr[s] = vd0 + vd1;
      Rr[s] = vd0 + vd2;
      sd += vd0;
      ss += vd3[k] + vd4[k];
      if (a.prow) {
        a.prow[(size_t)i * S + s] = vd0;
        a.prow[(size_t)(N + i) * S + s] = vd3[k] + vd4[k];
      }
      if (a.mrow) {
        a.mrow[(size_t)i * S + s] = vd2;
        a.mrow[(size_t)(N + i) * S + s] = vd1;
      }
      if (a.output_ud) {
        const T mtl = a.mlayout == 1 ? a.mt[(size_t)il * S + s] : a.mt[s];
        const T mtr = a.mlayout == 1 ? a.mt[(size_t)ir * S + s] : a.mt[s];
        const T pbl = Bl[s], pbr = Br[s];
        const T invl = pbl != NI ? xexp2(rml + mtl - pbl) : T(0);
        const T invr = pbr != NI ? xexp2(rmr + mtr - pbr) : T(0);
        const T udl = vd2 * invl, udr = vd1 * invr;
        a.ud[(size_t)i * S + s] = udl;
        a.ud[(size_t)(N + i) * S + s] = udr;
        sul += udl;
        sur += udr;
        if (a.side_thr > 0.0) {
          bl += udl < T(0) ? -udl : udl;
          br += udr < T(0) ? -udr : udr;
        } else {
          bl = tmax(bl, udl < T(0) ? -udl : udl);
          br = tmax(br, udr < T(0) ? -udr : udr);
        }
      } else {
        a.gPl[(size_t)i * S + s] = vd2;
        a.gPr[(size_t)i * S + s] = vd1;
      }
    }
  }
  __syncthreads();
  // speciation terms land in the children's columns (each column has one parent)
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    if (c1v[k] >= 0) {
      Lr[c1v[k]] += vd3[k];
      Rr[c1v[k]] += vd4[k];
    }
    if (c2v[k] >= 0) {
      Rr[c2v[k]] += vd3[k];
      Lr[c2v[k]] += vd4[k];
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      sideL[s] = Lr[s];
      sideR[s] = Rr[s];
    }
  }
  if (a.psum) {
    const T tsd = block_sum(sd, red);
    const T tss = block_sum(ss, red);
    if (threadIdx.x == 0) {
      a.psum[i] = tsd;
      a.psum[N + i] = tss;
    }
  }
  if (a.output_ud) {
    const T tl = block_sum(sul, red);
    const T tr = block_sum(sur, red);
    T ql, qr;
    if (a.side_thr > 0.0) {
      ql = block_sum(bl, red);
      qr = block_sum(br, red);
    } else {
      ql = block_max(bl, red);
      qr = block_max(br, red);
    }
    if (threadIdx.x == 0) {
      a.A[i] = tl;
      a.A[N + i] = tr;
      if (a.side_active) {
        if (a.side_thr > 0.0) {
          a.side_active[i] = (double)ql > a.side_thr;
          a.side_active[N + i] = (double)qr > a.side_thr;
        } else {
          a.side_active[i] = ql != T(0);
          a.side_active[N + i] = qr != T(0);
        }
      }
    }
  }
}

// ---- Pibar VJP through the subtree sums ----------------------------------------------------------

template <typename T>
struct PvArgs {
  int S, use_col;
  long long N;
  const T *Pi, *col, *A, *rowmax;
  T* ud;
  const uint8_t *side_active, *active;
  const int64_t *sl, *sr, *red_idx;
  T* contrib;
};

template <typename T, int CPT>
__global__ __launch_bounds__(NT) void pibar_vjp_kernel(OpsTree t, PvArgs<T> a) {
  extern __shared__ unsigned char smraw[];
  T* U = reinterpret_cast<T*>(smraw);
  T* Up = U + t.S;
  __shared__ T red[NW];
  const int S = a.S;
  const long long row = blockIdx.x;
  const long long si = row < a.N ? row : row - a.N;
  T* crow = a.contrib + (size_t)row * S;
  bool go = a.side_active ? a.side_active[row] != 0 : true;
  if (go && a.active) go = a.active[a.red_idx[si]] != 0;
  if (!go) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = threadIdx.x + k * NT;
      if (s < S) crow[s] = 0;
    }
    return;
  }
  const long long child = row < a.N ? a.sl[si] : a.sr[si];
  T* udr = a.ud + (size_t)row * S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) U[s] = udr[s];
  }
  __syncthreads();
  subtree_scan(t, U, Up, red);
  const T A = a.A[row];
  const T rms = msafe(a.rowmax[child]);
  const T* pr = a.Pi + (size_t)child * S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      udr[s] = subtree_of(t, Up, s);
      const T pp = xexp2((a.use_col ? a.col[s] + pr[s] : pr[s]) - rms);
      crow[s] = pp * complement_of(t, Up, s, A);
    }
  }
}

// ---- fixed-order row accumulation -------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(256) void scatter_add_kernel(int S, long long n, const T* src, const int* order,
                                                          const int64_t* keys, T* dst, long long dst_stride) {
  const long long k = blockIdx.x;
  const int s = blockIdx.y * 256 + threadIdx.x;
  if (s >= S) return;
  const long long key = keys[k];
  if (key < 0 || (k > 0 && keys[k - 1] == key)) return;
  long long e = k + 1;  // end of the run of this key (the same for every thread)
  while (e < n && keys[e] == key) ++e;
  // the run's rows added in order; the loads of eight rows are issued before their adds
  T acc = 0;
  long long j = k;
  for (; j + 8 <= e; j += 8) {
    T x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = src[(size_t)order[j + i] * S + s];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += x[i];
  }
  for (; j < e; ++j) acc += src[(size_t)order[j] * S + s];
  dst[(size_t)(key * dst_stride) + s] += acc;
}

constexpr int SUM_CHUNK = 64;

// Sum over rows r0 <= r < r1 of column s of a row-major block with S columns,
// added in row order in float64 (with a second block B, each row's A + B is
// formed first).  The loads of eight rows are issued before their adds: the
// adds keep their order, so the sum is the one of the plain loop.
template <typename T>
__device__ __forceinline__ double col_sum(const T* A, const T* B, int S, long long r0, long long r1, int s) {
  double acc = 0.0;
  long long r = r0;
  for (; r + 8 <= r1; r += 8) {
    T x[8], y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = A[(size_t)(r + i) * S + s];
    if (B) {
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = B[(size_t)(r + i) * S + s];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc += (double)x[i] + (double)y[i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc += (double)x[i];
    }
  }
  for (; r < r1; ++r) {
    double x = (double)A[(size_t)r * S + s];
    if (B) x += (double)B[(size_t)r * S + s];
    acc += x;
  }
  return acc;
}

// Sum over chunks c < n of work[c * S + s], in chunk order, eight loads ahead.
__device__ __forceinline__ double chunk_sum(const double* work, int S, int n, int s) {
  double acc = 0.0;
  int c = 0;
  for (; c + 8 <= n; c += 8) {
    double x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = work[(size_t)(c + i) * S + s];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += x[i];
  }
  for (; c < n; ++c) acc += work[(size_t)c * S + s];
  return acc;
}

template <typename T>
__global__ __launch_bounds__(256) void rows_sum_stage1(int S, long long n, const T* src, double* work) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s >= S) return;
  const long long r0 = (long long)blockIdx.y * SUM_CHUNK;
  const long long r1 = min(n, r0 + SUM_CHUNK);
  work[(size_t)blockIdx.y * S + s] = col_sum<T>(src, nullptr, S, r0, r1, s);
}

// One chunk or fewer rows: both stages in one launch (same sums).
template <typename T>
__global__ __launch_bounds__(256) void rows_sum_single(int S, long long n, const T* src, T* dst) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s >= S) return;
  const double acc = col_sum<T>(src, nullptr, S, 0, n, s);
  dst[s] = (T)((double)dst[s] + acc);
}

// Column sums of up to 8 row blocks in one launch (grid z = block): row chunk
// y of block j, summed in row order in float64; one chunk writes the result,
// more write partials that rows_sum_multi_stage2 adds in chunk order.
struct RsmArgs {
  int S, m, chunks;
  long long n;
  const void* a[8];
  const void* b[8];  // optional second addend of each block
};

template <typename T>
__global__ __launch_bounds__(256) void rows_sum_multi_stage1(RsmArgs p, double* work, T* out) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s >= p.S) return;
  const int j = blockIdx.z, c = blockIdx.y;
  const T* A = static_cast<const T*>(p.a[j]);
  const T* B = static_cast<const T*>(p.b[j]);
  const long long r0 = (long long)c * SUM_CHUNK, r1 = min(p.n, r0 + SUM_CHUNK);
  const double acc = col_sum<T>(A, B, p.S, r0, r1, s);
  if (p.chunks == 1)
    out[(size_t)j * p.S + s] = (T)acc;
  else
    work[((size_t)j * p.chunks + c) * p.S + s] = acc;
}

template <typename T>
__global__ __launch_bounds__(256) void rows_sum_multi_stage2(RsmArgs p, const double* work, T* out) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s >= p.S) return;
  const int j = blockIdx.z;
  out[(size_t)j * p.S + s] = (T)chunk_sum(work + (size_t)j * p.chunks * p.S, p.S, p.chunks, s);
}

// Column sums of up to 8 row blocks, each added into its own accumulator row:
// block j has n[j] rows of k[j] <= 4 addends (each row's addends summed first,
// in order), summed in row order in float64.  Blocks of one chunk add into
// their accumulator in stage 1 when no block has more (one launch); otherwise
// stage 1 writes every block's chunk partials and stage 2 adds them in chunk
// order, so each accumulator gets dst + sum, as rows_sum_single /
// rows_sum_stage2 form it.
struct RsaArgs {
  int S, m, chunks;  // chunks: the most any block has
  long long n[8];
  int k[8];
  const void* a[8][4];
  void* dst[8];
};

template <typename T>
__device__ __forceinline__ double col_sum_k(const RsaArgs& p, int j, long long r0, long long r1, int s) {
  const int S = p.S;
  const T* A0 = static_cast<const T*>(p.a[j][0]);
  if (p.k[j] == 1) return col_sum<T>(A0, nullptr, S, r0, r1, s);
  if (p.k[j] == 2) return col_sum<T>(A0, static_cast<const T*>(p.a[j][1]), S, r0, r1, s);
  const T* A1 = static_cast<const T*>(p.a[j][1]);
  const T* A2 = static_cast<const T*>(p.a[j][2]);
  const T* A3 = p.k[j] > 3 ? static_cast<const T*>(p.a[j][3]) : nullptr;
  double acc = 0.0;
  long long r = r0;
  for (; r + 4 <= r1; r += 4) {
    T x[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const size_t o = (size_t)(r + i) * S + s;
      x[i][0] = A0[o];
      x[i][1] = A1[o];
      x[i][2] = A2[o];
      x[i][3] = A3 ? A3[o] : T(0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      double v = (double)x[i][0] + (double)x[i][1] + (double)x[i][2];
      if (A3) v += (double)x[i][3];
      acc += v;
    }
  }
  for (; r < r1; ++r) {
    const size_t o = (size_t)r * S + s;
    double v = (double)A0[o] + (double)A1[o] + (double)A2[o];
    if (A3) v += (double)A3[o];
    acc += v;
  }
  return acc;
}

template <typename T>
__global__ __launch_bounds__(256) void rows_sum_accum_stage1(RsaArgs p, double* work) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  const int j = blockIdx.z, c = blockIdx.y;
  if (s >= p.S) return;
  const long long r0 = (long long)c * SUM_CHUNK, r1 = min(p.n[j], r0 + SUM_CHUNK);
  if (p.chunks == 1) {
    T* D = static_cast<T*>(p.dst[j]);
    D[s] = (T)((double)D[s] + col_sum_k<T>(p, j, 0, p.n[j], s));
    return;
  }
  if (r0 >= p.n[j]) return;
  work[((size_t)j * p.chunks + c) * p.S + s] = col_sum_k<T>(p, j, r0, r1, s);
}

template <typename T>
__global__ __launch_bounds__(256) void rows_sum_accum_stage2(RsaArgs p, const double* work) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  const int j = blockIdx.z;
  if (s >= p.S || p.n[j] <= 0) return;
  const int nc = (int)((p.n[j] + SUM_CHUNK - 1) / SUM_CHUNK);
  T* D = static_cast<T*>(p.dst[j]);
  D[s] = (T)((double)D[s] + chunk_sum(work + (size_t)j * p.chunks * p.S, p.S, nc, s));
}

template <typename T>
__global__ __launch_bounds__(256) void rows_sum_stage2(int S, int n_chunks, const double* work, T* dst) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s >= S) return;
  const double acc = chunk_sum(work, S, n_chunks, s);
  dst[s] = (T)((double)dst[s] + acc);
}

}  // namespace kbo

// Device scratch of kb_estep_vjp_noalloc: the [G, S] float64 grad_col
// contributions.  Each GPU holds its own copy for the life of the process; in
// host code its name is only a symbol handle, so the address used in launches
// comes from hipGetSymbolAddress (scratch_on_current_device below).
static __device__ __align__(256) double scratch[KB_ESTEP_VJP_NOALLOC_MAX];

// =====================================================================================
// host side
// =====================================================================================

namespace {

using namespace kbo_host;

// Address of `scratch` on the current device, looked up once per device.
int scratch_on_current_device(double** out) {
  static std::mutex mu;
  static std::vector<double*> addr;  // by device ordinal; nullptr until looked up
  int dev = -1;
  KBO_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  if ((int)addr.size() <= dev) addr.resize(dev + 1, nullptr);
  if (!addr[dev]) {
    void* p = nullptr;
    KBO_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    addr[dev] = static_cast<double*>(p);
  }
  *out = addr[dev];
  return 0;
}


int put(int** dst, const std::vector<int>& v) {
  *dst = nullptr;
  KBO_HIP(hipMalloc((void**)dst, std::max<size_t>(1, v.size()) * sizeof(int)));
  if (!v.empty()) KBO_HIP(hipMemcpy(*dst, v.data(), v.size() * sizeof(int), hipMemcpyHostToDevice));
  return 0;
}

}  // namespace

extern "C" {

int kb_tree_create(int32_t S, const int64_t* parent, const int64_t* child1, const int64_t* child2, kb_tree** out) {
  if (!out || !parent || !child1 || !child2) return kb::set_error(KB_ERR_ARG, "null argument");
  *out = nullptr;
  if (S < 1 || S > 8192) return kb::set_error(KB_ERR_ARG, "S=%d outside [1, 8192]", S);
  std::vector<int> par(S), c1(S), c2(S);
  int root = -1;
  for (int s = 0; s < S; ++s) {
    const int64_t p = parent[s];
    if (p < 0 || p >= S) {
      if (root >= 0) return kb::set_error(KB_ERR_ARG, "node_parent has more than one root (%d, %d)", root, s);
      root = s;
      par[s] = -1;
    } else {
      par[s] = (int)p;
    }
    c1[s] = (child1[s] >= 0 && child1[s] < S) ? (int)child1[s] : -1;
    c2[s] = (child2[s] >= 0 && child2[s] < S) ? (int)child2[s] : -1;
  }
  if (root < 0) return kb::set_error(KB_ERR_ARG, "node_parent has no root");
  for (int s = 0; s < S; ++s) {
    for (int c : {c1[s], c2[s]})
      if (c >= 0 && par[c] != s)
        return kb::set_error(KB_ERR_ARG, "node_child of %d is %d but node_parent[%d] = %d", s, c, c, par[c]);
    if (par[s] >= 0 && c1[par[s]] != s && c2[par[s]] != s)
      return kb::set_error(KB_ERR_ARG, "node %d is not a child of its parent %d", s, par[s]);
  }
  // preorder DFS (child1 first), Euler tour, depths
  std::vector<int> pcol, ppos(S, -1), pend(S, 0), tin(S, 0), ev, depth(S, 0);
  pcol.reserve(S);
  ev.reserve(2 * S);
  std::vector<std::pair<int, int>> stack;  // (node, state) 0: enter, 1: exit
  stack.push_back({root, 0});
  while (!stack.empty()) {
    auto [n, state] = stack.back();
    stack.pop_back();
    if (state == 0) {
      if (ppos[n] >= 0) return kb::set_error(KB_ERR_ARG, "species tree has a cycle at node %d", n);
      ppos[n] = (int)pcol.size();
      pcol.push_back(n);
      tin[n] = (int)ev.size();
      ev.push_back(n << 1);
      stack.push_back({n, 1});
      if (c2[n] >= 0) {
        depth[c2[n]] = depth[n] + 1;
        stack.push_back({c2[n], 0});
      }
      if (c1[n] >= 0) {
        depth[c1[n]] = depth[n] + 1;
        stack.push_back({c1[n], 0});
      }
    } else {
      pend[n] = (int)pcol.size();
      ev.push_back((n << 1) | 1);
    }
  }
  if ((int)pcol.size() != S)
    return kb::set_error(KB_ERR_ARG, "species tree is not connected (%zu of %d nodes reachable)", pcol.size(), S);
  int max_d = 0;
  for (int s = 0; s < S; ++s) max_d = std::max(max_d, depth[s]);
  std::vector<int> lvl_ptr(max_d + 2, 0), lvl_node(S);
  for (int s = 0; s < S; ++s) ++lvl_ptr[depth[s] + 1];
  for (int d = 0; d <= max_d; ++d) lvl_ptr[d + 1] += lvl_ptr[d];
  {
    std::vector<int> fill(lvl_ptr.begin(), lvl_ptr.end() - 1);
    for (int s = 0; s < S; ++s) lvl_node[fill[depth[s]]++] = s;
  }
  // preorder-position tables of the contiguous-ownership sweeps
  std::vector<int> pc1(S), pc2(S), pnex(S), ppost;
  ppost.reserve(S);
  for (int i = 0; i < S; ++i) {
    const int n = pcol[i];
    pc1[i] = c1[n] >= 0 ? ppos[c1[n]] : -1;
    pc2[i] = c2[n] >= 0 ? ppos[c2[n]] : -1;
    pnex[i] = tin[n] - i;
  }
  for (int e : ev)
    if (e & 1) ppost.push_back(ppos[e >> 1]);
  kb_tree* t = new kb_tree();
  t->S = S;
  t->n_levels = max_d + 1;
  int rc = 0;
  rc |= put(&t->par, par);
  rc |= put(&t->c1, c1);
  rc |= put(&t->c2, c2);
  rc |= put(&t->ev, ev);
  rc |= put(&t->tin, tin);
  rc |= put(&t->pcol, pcol);
  rc |= put(&t->ppos, ppos);
  rc |= put(&t->pend, pend);
  rc |= put(&t->lvl_ptr, lvl_ptr);
  rc |= put(&t->lvl_node, lvl_node);
  rc |= put(&t->pc1, pc1);
  rc |= put(&t->pc2, pc2);
  rc |= put(&t->pnex, pnex);
  rc |= put(&t->ppost, ppost);
  if (rc) {
    kb_tree_destroy(t);
    return KB_ERR_HIP;
  }
  *out = t;
  return 0;
}

void kb_tree_destroy(kb_tree* t) {
  if (!t) return;
  for (int* p : {t->par, t->c1, t->c2, t->ev, t->tin, t->pcol, t->ppos, t->pend, t->lvl_ptr, t->lvl_node, t->pc1,
                 t->pc2, t->pnex, t->ppost})
    if (p) (void)hipFree(p);
  delete t;
}

int kb_ops_max_states(int dtype) {
  // wave_step / wave_backward use 4 S elements of LDS per row
  const size_t per = 4 * elem_size(dtype);
  size_t s = LDS_BYTES / per;
  return (int)std::min<size_t>(8192, s);
}

int kb_estep(const kb_tree* tr, const kb_estep_io* io, void* stream) {
  if (!tr || !io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->G < 0) return kb::set_error(KB_ERR_ARG, "G must be non-negative");
  if (io->mode == 1 && (io->max_iter < 1 || !(io->tol > 0.0)))
    return kb::set_error(KB_ERR_ARG, "max_iter must be >= 1 and tol > 0");
  if (io->G == 0) return 0;
  const int S = tr->S;
  const size_t lds = (size_t)2 * S * sizeof(double);
  if (int rc = check_lds(lds, S, KB_F64)) return rc;
  const kbo::OpsTree t = tr->dev();
  KBO_DISPATCH(io->dtype, S, {
    kbo::EsArgs<T> a{io->G, S, io->mode, io->use_col_weights, io->max_iter, io->tol,
                     (const T*)io->E, (const T*)io->log_pS, (const T*)io->log_pD, (const T*)io->log_pL,
                     (const T*)io->max_coupling, (const T*)io->col_log_probs,
                     (T*)io->E_out, (T*)io->E_s1, (T*)io->E_s2, (T*)io->Ebar, (T*)io->max_diff, io->n_iter};
    auto k = kbo::estep_kernel<T, CPT>;
    if (int rc = set_lds(k, lds)) return rc;
    hipLaunchKernelGGL(k, dim3(io->G), dim3(kbo::NT), lds, st_of(stream), t, a);
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"

namespace {

// The E-step VJP launches with `work` ([G, S] float64) as the grad_col staging rows.
int estep_vjp_launch(const kb_tree* tr, const kb_estep_vjp_io* io, double* work, void* stream) {
  const int S = tr->S;
  const size_t lds = (size_t)2 * S * sizeof(double);
  if (int rc = check_lds(lds, S, KB_F64)) return rc;
  const kbo::OpsTree t = tr->dev();
  KBO_DISPATCH(io->dtype, S, {
    kbo::EvArgs<T> a{io->G, S, io->use_col_weights,
                     (const T*)io->E, (const T*)io->E_new, (const T*)io->E_s1, (const T*)io->E_s2, (const T*)io->Ebar,
                     (const T*)io->log_pS, (const T*)io->log_pD, (const T*)io->log_pL, (const T*)io->col_log_probs,
                     (const T*)io->g_E_new, (const T*)io->g_E_s1, (const T*)io->g_E_s2, (const T*)io->g_Ebar,
                     (T*)io->grad_E, (T*)io->grad_log_pS, (T*)io->grad_log_pD, (T*)io->grad_log_pL,
                     (T*)io->grad_max_coupling, work};
    auto k = kbo::estep_vjp_kernel<T, CPT>;
    if (int rc = set_lds(k, lds)) return rc;
    hipLaunchKernelGGL(k, dim3(io->G), dim3(kbo::NT), lds, st_of(stream), t, a);
    // grad_col += sum over item rows of the per-row contributions (fixed row order)
    hipLaunchKernelGGL((kbo::rows_sum_stage2<T>), dim3((S + 255) / 256), dim3(256), 0, st_of(stream), S, io->G,
                       (const double*)work, (T*)io->grad_col_log_probs);
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

}  // namespace

namespace {
// Chains of float sweeps run the linear-space preorder-ownership kernel (three
// LDS rows of NT * CPT + 64 floats; its set-up -- tables, linear constants, the
// row permuted through LDS -- pays off over several sweeps); single sweeps and
// float64 rows the log-space Euler-tour one.  A chain agrees with the same
// sweeps launched one at a time to float32 rounding.
template <typename T, int CPT>
int launch_wave_step(const kbo::OpsTree& t, const kbo::WsArgs<T>& a, int W, size_t lds, hipStream_t st) {
  if constexpr (std::is_same_v<T, float>) {
    if (a.n_sweeps > 1) {
      const size_t lds_lin = (size_t)3 * (kbo::NT * CPT + 64) * sizeof(float);
      auto k = kbo::wave_step_lin_kernel<CPT>;
      if (int rc = set_lds(k, lds_lin)) return rc;
      hipLaunchKernelGGL(k, dim3(W), dim3(kbo::NT), lds_lin, st, t, a);
      return 0;
    }
  }
  auto k = kbo::wave_step_kernel<T, CPT>;
  if (int rc = set_lds(k, lds)) return rc;
  hipLaunchKernelGGL(k, dim3(W), dim3(kbo::NT), lds, st, t, a);
  return 0;
}

// float32 rows of the per-call wave backward run the preorder-ownership kernel
template <typename T, int CPT>
int launch_wave_bwd(const kbo::OpsTree& t, const kbo::WbArgs<T>& a, int W, size_t lds, hipStream_t st) {
  if constexpr (std::is_same_v<T, float>) {
    const size_t lds_pre = (size_t)4 * (kbo::NT * CPT + 64) * sizeof(float);
    auto k = kbo::wave_bwd_pre_kernel<CPT>;
    if (int rc = set_lds(k, lds_pre)) return rc;
    hipLaunchKernelGGL(k, dim3(W), dim3(kbo::NT), lds_pre, st, t, a);
    return 0;
  }
  auto k = kbo::wave_bwd_kernel<T, CPT>;
  if (int rc = set_lds(k, lds)) return rc;
  hipLaunchKernelGGL(k, dim3(W), dim3(kbo::NT), lds, st, t, a);
  return 0;
}

}  // namespace

extern "C" {

int kb_estep_vjp(const kb_tree* tr, const kb_estep_vjp_io* io, void* stream) {
  if (!tr || !io || !io->work) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->G <= 0) return kb::set_error(KB_ERR_ARG, "G must be positive");
  return estep_vjp_launch(tr, io, io->work, stream);
}

int kb_estep_vjp_noalloc(const kb_tree* tr, const kb_estep_vjp_io* io, void* stream) {
  if (!tr || !io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (io->work) return kb::set_error(KB_ERR_ARG, "kb_estep_vjp_noalloc takes no work buffer (io->work must be NULL)");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->G <= 0) return kb::set_error(KB_ERR_ARG, "G must be positive");
  if ((int64_t)io->G * tr->S > (int64_t)KB_ESTEP_VJP_NOALLOC_MAX)
    return kb::set_error(KB_ERR_ARG, "kb_estep_vjp_noalloc: G * S = %lld exceeds its scratch of %d doubles",
                         (long long)io->G * tr->S, (int)KB_ESTEP_VJP_NOALLOC_MAX);
  double* work = nullptr;
  if (int rc = scratch_on_current_device(&work)) return rc;
  return estep_vjp_launch(tr, io, work, stream);
}

int kb_wave_step(const kb_tree* tr, const kb_wave_step_io* io, void* stream) {
  if (!tr || !io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->S != tr->S) return kb::set_error(KB_ERR_ARG, "S=%d does not match the tree (%d)", io->S, tr->S);
  if (io->W <= 0) return 0;
  const int S = io->S;
  const size_t lds = (size_t)4 * S * elem_size(io->dtype);
  if (int rc = check_lds(lds, S, io->dtype)) return rc;
  const kbo::OpsTree t = tr->dev();
  KBO_DISPATCH(io->dtype, S, {
    kbo::WsArgs<T> a{S, io->W, io->use_col_weights, io->use_leaf_index, io->store_final_pibar,
                     io->n_sweeps > 1 ? io->n_sweeps : 1, io->ws, io->pi_ws,
                     io->const_stride, (const T*)io->Pi_in, (T*)io->Pi_out, (T*)io->Pibar, (T*)io->pibar_row_max,
                     io->pi_residual, (const T*)io->dts, (const T*)io->max_coupling, (const T*)io->DL,
                     (const T*)io->Ebar, (const T*)io->E, (const T*)io->SL1, (const T*)io->SL2,
                     (const T*)io->col_log_probs, io->item_idx, io->leaf_state, (const T*)io->leaf_logp};
    if (int rc = launch_wave_step<T, CPT>(t, a, io->W, lds, st_of(stream))) return rc;
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_leaf_init(const kb_leaf_init_io* io, void* stream) {
  if (!io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->W <= 0) return 0;
  if (!io->node_child1 || !io->node_child2) return kb::set_error(KB_ERR_ARG, "node_child1/2 are required");
  dim3 g(io->W, (io->S + 255) / 256);
  if (io->dtype == KB_F64) {
    using T = double;
    kbo::LiArgs<T> a{io->S, io->W, io->use_col_weights, io->ws, io->const_stride, (T*)io->Pi_out,
                     (const T*)io->max_coupling, (const T*)io->DL, (const T*)io->Ebar, (const T*)io->E,
                     (const T*)io->SL1, (const T*)io->SL2, (const T*)io->col_log_probs, io->subtree_start,
                     io->subtree_end, io->item_idx, io->leaf_state, io->node_child1, io->node_child2,
                     (const T*)io->leaf_logp};
    hipLaunchKernelGGL(kbo::leaf_init_kernel<T>, g, dim3(256), 0, st_of(stream), a);
  } else {
    using T = float;
    kbo::LiArgs<T> a{io->S, io->W, io->use_col_weights, io->ws, io->const_stride, (T*)io->Pi_out,
                     (const T*)io->max_coupling, (const T*)io->DL, (const T*)io->Ebar, (const T*)io->E,
                     (const T*)io->SL1, (const T*)io->SL2, (const T*)io->col_log_probs, io->subtree_start,
                     io->subtree_end, io->item_idx, io->leaf_state, io->node_child1, io->node_child2,
                     (const T*)io->leaf_logp};
    hipLaunchKernelGGL(kbo::leaf_init_kernel<T>, g, dim3(256), 0, st_of(stream), a);
  }
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_dts_forward(const kb_dts_io* io, void* stream) {
  if (!io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->W <= 0) return 0;
  if (!io->node_child1 || !io->node_child2) return kb::set_error(KB_ERR_ARG, "node_child1/2 are required");
  const int S = io->S;
  KBO_DISPATCH(io->dtype, S, {
    kbo::DtsArgs<T> a{S, io->W, io->param_by_state, io->item_offset, io->param_row_stride, (const T*)io->Pi,
                      (const T*)io->Pibar, (const T*)io->log_split_probs, (const T*)io->log_pD,
                      (const T*)io->log_pS, io->sl, io->sr, io->item_idx, io->node_child1, io->node_child2,
                      io->split_ptr, io->split_order, io->active, (T*)io->out};
    hipLaunchKernelGGL((kbo::dts_kernel<T, CPT>), dim3(io->W), dim3(kbo::NT), 0, st_of(stream), a);
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_active_mask(int32_t dtype, int32_t W, int32_t S, int64_t row_stride, const void* rhs, float threshold,
                   int32_t strict, uint8_t* active, void* stream) {
  if (W < 0 || S < 0) return kb::set_error(KB_ERR_ARG, "bad sizes");
  if (W == 0) return 0;
  if (!rhs || !active) return kb::set_error(KB_ERR_ARG, "null argument");
  if (dtype == KB_F64)
    hipLaunchKernelGGL(kbo::active_kernel<double>, dim3(W), dim3(256), 0, st_of(stream), S, (long long)row_stride,
                       (const double*)rhs, threshold, strict, active);
  else if (dtype == KB_BF16)
    hipLaunchKernelGGL(kbo::active_kernel<__hip_bfloat16>, dim3(W), dim3(256), 0, st_of(stream), S,
                       (long long)row_stride, (const __hip_bfloat16*)rhs, threshold, strict, active);
  else if (dtype == KB_F32)
    hipLaunchKernelGGL(kbo::active_kernel<float>, dim3(W), dim3(256), 0, st_of(stream), S, (long long)row_stride,
                       (const float*)rhs, threshold, strict, active);
  else
    return kb::set_error(KB_ERR_ARG, "active mask supports float32, float64 and bfloat16");
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_wave_backward(const kb_tree* tr, const kb_wave_bwd_io* io, void* stream) {
  if (!tr || !io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->S != tr->S) return kb::set_error(KB_ERR_ARG, "S=%d does not match the tree (%d)", io->S, tr->S);
  if (io->n_terms < 0) return kb::set_error(KB_ERR_ARG, "neumann_terms must be non-negative");
  if (io->W <= 0) return 0;
  const int S = io->S;
  const size_t lds = (size_t)4 * S * elem_size(io->dtype);
  if (int rc = check_lds(lds, S, io->dtype)) return rc;
  const kbo::OpsTree t = tr->dev();
  KBO_DISPATCH(io->dtype, S, {
    kbo::WbArgs<T> a{S, io->W, io->n_terms, io->const_layout, io->leaf_mode, io->use_leaf_index,
                     io->use_col_weights, io->ws, (const T*)io->Pi, (const T*)io->Pibar, (const T*)io->pibar_row_max,
                     (const T*)io->dts, (const T*)io->rhs, (const T*)io->initial_v, io->active, (const T*)io->max_coupling, (const T*)io->DL,
                     (const T*)io->Ebar, (const T*)io->E, (const T*)io->SL1, (const T*)io->SL2,
                     (const T*)io->col_log_probs, io->item_idx, io->leaf_state, (const T*)io->leaf_logp,
                     (const T*)io->leaf_term, (T*)io->v, (T*)io->aw0, (T*)io->aw1, (T*)io->aw2, (T*)io->aw345,
                     (T*)io->aw3, (T*)io->aw4, (T*)io->col_rows, io->relres};
    if (int rc = launch_wave_bwd<T, CPT>(t, a, io->W, lds, st_of(stream))) return rc;
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_dts_cross_backward(const kb_dts_cross_io* io, void* stream) {
  if (!io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->N <= 0) return 0;
  if (!io->node_child1 || !io->node_child2) return kb::set_error(KB_ERR_ARG, "node_child1/2 are required");
  if (!io->side_rows) return kb::set_error(KB_ERR_ARG, "side_rows is required");
  if (io->output_ud && (!io->ud || !io->A || !io->mt || !io->pibar_row_max))
    return kb::set_error(KB_ERR_ARG, "output_ud needs ud, A, mt and pibar_row_max");
  if (!io->output_ud && (!io->grad_Pibar_l || !io->grad_Pibar_r))
    return kb::set_error(KB_ERR_ARG, "grad_Pibar_l / grad_Pibar_r are required without output_ud");
  if ((io->param_layout >= 2 || io->mt_layout == 1) && !io->item_idx)
    return kb::set_error(KB_ERR_ARG, "item-indexed layouts need item_idx");
  const int S = io->S;
  const size_t lds = (size_t)2 * S * elem_size(io->dtype);
  if (int rc = check_lds(lds, S, io->dtype)) return rc;
  KBO_DISPATCH(io->dtype, S, {
    kbo::DcArgs<T> a{S, io->param_layout, io->mt_layout, io->output_ud, io->skip_inactive_ud_zero, io->N, io->ws,
                     io->side_threshold, (const T*)io->Pi, (const T*)io->Pibar, (const T*)io->v, io->active, io->sl,
                     io->sr, io->reduce_idx, io->item_idx, io->node_child1, io->node_child2, (const T*)io->wlsp, (const T*)io->log_pD,
                     (const T*)io->log_pS, (const T*)io->mt, (const T*)io->pibar_row_max, (T*)io->side_rows,
                     (T*)io->ud, (T*)io->A, io->side_active, (T*)io->grad_Pibar_l, (T*)io->grad_Pibar_r,
                     (T*)io->param_rows, (T*)io->param_sums, (T*)io->mt_rows};
    auto k = kbo::dts_cross_kernel<T, CPT>;
    if (int rc = set_lds(k, lds)) return rc;
    hipLaunchKernelGGL(k, dim3((unsigned)io->N), dim3(kbo::NT), lds, st_of(stream), a);
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_pibar_vjp(const kb_tree* tr, const kb_pibar_vjp_io* io, void* stream) {
  if (!tr || !io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->S != tr->S) return kb::set_error(KB_ERR_ARG, "S=%d does not match the tree (%d)", io->S, tr->S);
  if (io->N <= 0) return 0;
  if (io->active && !io->reduce_idx) return kb::set_error(KB_ERR_ARG, "reduce_idx is required with active");
  const int S = io->S;
  const size_t lds = (size_t)2 * S * elem_size(io->dtype);
  if (int rc = check_lds(lds, S, io->dtype)) return rc;
  const kbo::OpsTree t = tr->dev();
  KBO_DISPATCH(io->dtype, S, {
    kbo::PvArgs<T> a{S, io->use_col_weights, io->N, (const T*)io->Pi, (const T*)io->col_log_probs, (const T*)io->A,
                     (const T*)io->pibar_row_max, (T*)io->ud, io->side_active, io->active, io->sl, io->sr,
                     io->reduce_idx, (T*)io->contrib};
    auto k = kbo::pibar_vjp_kernel<T, CPT>;
    if (int rc = set_lds(k, lds)) return rc;
    hipLaunchKernelGGL(k, dim3((unsigned)(2 * io->N)), dim3(kbo::NT), lds, st_of(stream), t, a);
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_rows_scatter_add(int32_t dtype, int32_t S, int64_t n, const void* src, const int32_t* order,
                        const int64_t* keys_sorted, void* dst, int64_t dst_stride, void* stream) {
  if (n <= 0 || S <= 0) return 0;
  if (!src || !order || !keys_sorted || !dst) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(dtype)) return rc;
  dim3 g((unsigned)n, (S + 255) / 256);
  if (dtype == KB_F64)
    hipLaunchKernelGGL(kbo::scatter_add_kernel<double>, g, dim3(256), 0, st_of(stream), S, (long long)n,
                       (const double*)src, order, keys_sorted, (double*)dst, (long long)dst_stride);
  else
    hipLaunchKernelGGL(kbo::scatter_add_kernel<float>, g, dim3(256), 0, st_of(stream), S, (long long)n,
                       (const float*)src, order, keys_sorted, (float*)dst, (long long)dst_stride);
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_rows_sum_multi(int32_t dtype, int32_t S, int64_t n, int32_t m, const void* const* a, const void* const* b,
                      void* out, double* work, void* stream) {
  if (S <= 0 || m <= 0) return 0;
  if (m > 8) return kb::set_error(KB_ERR_ARG, "at most 8 row blocks per call (m=%d)", m);
  if (!a || !out) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(dtype)) return rc;
  kbo::RsmArgs p{};
  p.S = S;
  p.m = m;
  p.n = n;
  p.chunks = (int)std::max<int64_t>(1, (n + kbo::SUM_CHUNK - 1) / kbo::SUM_CHUNK);
  for (int j = 0; j < m; ++j) {
    if (!a[j] && n > 0) return kb::set_error(KB_ERR_ARG, "row block %d is null", j);
    p.a[j] = a[j];
    p.b[j] = b ? b[j] : nullptr;
  }
  if (p.chunks > 1 && !work) return kb::set_error(KB_ERR_ARG, "work is required for more than 64 rows");
  const dim3 g1((S + 255) / 256, p.chunks, m), g2((S + 255) / 256, 1, m);
  if (dtype == KB_F64) {
    hipLaunchKernelGGL(kbo::rows_sum_multi_stage1<double>, g1, dim3(256), 0, st_of(stream), p, work, (double*)out);
    if (p.chunks > 1)
      hipLaunchKernelGGL(kbo::rows_sum_multi_stage2<double>, g2, dim3(256), 0, st_of(stream), p, work, (double*)out);
  } else {
    hipLaunchKernelGGL(kbo::rows_sum_multi_stage1<float>, g1, dim3(256), 0, st_of(stream), p, work, (float*)out);
    if (p.chunks > 1)
      hipLaunchKernelGGL(kbo::rows_sum_multi_stage2<float>, g2, dim3(256), 0, st_of(stream), p, work, (float*)out);
  }
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_rows_sum_accum(int32_t dtype, int32_t S, int32_t m, const int64_t* n, const int32_t* k, const void* const* a,
                      void* const* dst, double* work, void* stream) {
  if (S <= 0 || m <= 0) return 0;
  if (m > 8) return kb::set_error(KB_ERR_ARG, "at most 8 row blocks per call (m=%d)", m);
  if (!n || !k || !a || !dst) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(dtype)) return rc;
  kbo::RsaArgs p{};
  p.S = S;
  p.m = m;
  p.chunks = 1;
  for (int j = 0; j < m; ++j) {
    if (n[j] < 0) return kb::set_error(KB_ERR_ARG, "row block %d has %lld rows", j, (long long)n[j]);
    if (k[j] < 1 || k[j] > 4) return kb::set_error(KB_ERR_ARG, "row block %d has %d addends (1..4)", j, k[j]);
    if (!dst[j]) return kb::set_error(KB_ERR_ARG, "row block %d has no accumulator", j);
    for (int i = 0; i < j; ++i)
      if (dst[i] == dst[j]) return kb::set_error(KB_ERR_ARG, "row blocks %d and %d share an accumulator", i, j);
    p.n[j] = n[j];
    p.k[j] = k[j];
    p.dst[j] = dst[j];
    for (int i = 0; i < k[j]; ++i) {
      if (!a[4 * j + i] && n[j] > 0) return kb::set_error(KB_ERR_ARG, "row block %d addend %d is null", j, i);
      p.a[j][i] = a[4 * j + i];
    }
    p.chunks = (int)std::max<int64_t>(p.chunks, (n[j] + kbo::SUM_CHUNK - 1) / kbo::SUM_CHUNK);
  }
  if (p.chunks > 1 && !work) return kb::set_error(KB_ERR_ARG, "work is required for blocks of more than 64 rows");
  const dim3 g1((S + 255) / 256, p.chunks, m), g2((S + 255) / 256, 1, m);
  if (dtype == KB_F64) {
    hipLaunchKernelGGL(kbo::rows_sum_accum_stage1<double>, g1, dim3(256), 0, st_of(stream), p, work);
    if (p.chunks > 1)
      hipLaunchKernelGGL(kbo::rows_sum_accum_stage2<double>, g2, dim3(256), 0, st_of(stream), p, (const double*)work);
  } else {
    hipLaunchKernelGGL(kbo::rows_sum_accum_stage1<float>, g1, dim3(256), 0, st_of(stream), p, work);
    if (p.chunks > 1)
      hipLaunchKernelGGL(kbo::rows_sum_accum_stage2<float>, g2, dim3(256), 0, st_of(stream), p, (const double*)work);
  }
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_rows_sum_into(int32_t dtype, int32_t S, int64_t n, const void* src, void* dst, double* work, void* stream) {
  if (n <= 0 || S <= 0) return 0;
  if (!src || !dst || !work) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(dtype)) return rc;
  const int chunks = (int)((n + kbo::SUM_CHUNK - 1) / kbo::SUM_CHUNK);
  dim3 g1((S + 255) / 256, chunks);
  if (chunks == 1) {  // one launch, same sum as the two stages
    if (dtype == KB_F64)
      hipLaunchKernelGGL(kbo::rows_sum_single<double>, dim3((S + 255) / 256), dim3(256), 0, st_of(stream), S,
                         (long long)n, (const double*)src, (double*)dst);
    else
      hipLaunchKernelGGL(kbo::rows_sum_single<float>, dim3((S + 255) / 256), dim3(256), 0, st_of(stream), S,
                         (long long)n, (const float*)src, (float*)dst);
  } else if (dtype == KB_F64) {
    hipLaunchKernelGGL(kbo::rows_sum_stage1<double>, g1, dim3(256), 0, st_of(stream), S, (long long)n,
                       (const double*)src, work);
    hipLaunchKernelGGL(kbo::rows_sum_stage2<double>, dim3((S + 255) / 256), dim3(256), 0, st_of(stream), S, chunks,
                       (const double*)work, (double*)dst);
  } else {
    hipLaunchKernelGGL(kbo::rows_sum_stage1<float>, g1, dim3(256), 0, st_of(stream), S, (long long)n,
                       (const float*)src, work);
    hipLaunchKernelGGL(kbo::rows_sum_stage2<float>, dim3((S + 255) / 256), dim3(256), 0, st_of(stream), S, chunks,
                       (const double*)work, (float*)dst);
  }
  KBO_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
