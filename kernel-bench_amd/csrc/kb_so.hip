// Second-order contractions of the backward maps for the exact Hessian-vector
// product: the launchers beneath the drop-in replacements of the reference's
// kbench/core/kernels/e_step_so.py, wave_so.py and dts_so.py (declarations and
// the reference function each replaces: include/kbench_ops.h).
//
// Each backward map is linear in its cotangent and nonlinear in its primal
// point; these kernels return its directional derivative along a primal
// tangent at a fixed cotangent.  The structure mirrors the first-order
// kernels: one 1024-thread workgroup per row, ancestor path sums by an
// Euler-tour prefix scan and subtree sums by a preorder prefix scan in LDS,
// scatters onto child columns written as gathers from the parent column
// (every column has one parent), cross-row accumulations emitted as rows and
// summed in a fixed order by the caller, float64 arithmetic inside.  The
// saved row maxima are frozen (every output is invariant to the row
// normaliser).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "kb_ops_common.hpp"

namespace kbo {

constexpr double LN2D = 0.6931471805599453;

template <typename T>
__device__ __forceinline__ double ld(const T* p, size_t i) {
  return (double)p[i];
}

template <typename C, typename T>
__device__ __forceinline__ C ldc(const T* p, size_t i) {
  return (C)p[i];
}

// ---- E-step ------------------------------------------------------------------------

template <typename T>
struct EsoArgs {
  int G, S, use_col;
  const T *E, *En, *Es1, *Es2, *Eb, *pS, *pD, *pL, *col, *gN, *gB;
  const T *dE, *dEn, *dEs1, *dEs2, *dEb, *dpS, *dpD, *dpL, *dcol;
  T *oE, *opS, *opD, *opL, *omc, *ocol;
};

// One workgroup per item row.  q_k = g_new 2^(t_k - E_new), dq_k = ln2 q_k (dt_k - dE_new);
// d_grad_E = 2 dq1 + dq2 + dq0[parent] + dr (tot - excl) + r (dtot - dexcl) with
// u = (q2 + g_ebar) / denom, du = (dq2 - u ddenom) / denom, excl = subtree sums of u.
template <typename T, int CPT, typename C = double>
__global__ __launch_bounds__(NT) void eso_kernel(OpsTree t, EsoArgs<T> a) {
  extern __shared__ double smd[];  // raw storage: C values
  const int S = t.S;
  C* X = reinterpret_cast<C*>(smd);       // dq0 by column
  C* EV = reinterpret_cast<C*>(smd) + S;  // 2S scan buffer
  __shared__ C red[NW];
  const C NI = ninf<C>();
  const size_t base = (size_t)blockIdx.x * S;
  C gE[CPT], wE[CPT], dwE[CPT], dq2[CPT], q2g[CPT];
  C lm = NI;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    gE[k] = dq2[k] = q2g[k] = dwE[k] = C(0);
    wE[k] = NI;
    if (s < S) {
      const size_t i = base + s;
      const C E = ldc<C>(a.E, i), En = ldc<C>(a.En, i), dE = ldc<C>(a.dE, i), dEn = ldc<C>(a.dEn, i), g = ldc<C>(a.gN, i);
      const C t0 = ldc<C>(a.pS, i) + ldc<C>(a.Es1, i) + ldc<C>(a.Es2, i);
      const C t1 = ldc<C>(a.pD, i) + C(2) * E;
      const C t2 = E + ldc<C>(a.Eb, i);
      const C t3 = ldc<C>(a.pL, i);
      const C dt0 = ldc<C>(a.dpS, i) + ldc<C>(a.dEs1, i) + ldc<C>(a.dEs2, i);
      const C dt1 = ldc<C>(a.dpD, i) + C(2) * dE;
      const C dt2 = dE + ldc<C>(a.dEb, i);
      const C dt3 = ldc<C>(a.dpL, i);
      C q[4] = {g * xexp2(t0 - En), g * xexp2(t1 - En), g * xexp2(t2 - En), g * xexp2(t3 - En)};
      const C dt[4] = {dt0, dt1, dt2, dt3};
      C dq[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (q[j] != q[j]) q[j] = C(0);  // 0 * inf
        dq[j] = q[j] != C(0) ? (C)LN2D * q[j] * (dt[j] - dEn) : C(0);
      }
      a.opS[i] = (T)dq[0];
      a.opD[i] = (T)dq[1];
      a.opL[i] = (T)dq[3];
      a.omc[i] = (T)dq[2];
      X[s] = dq[0];
      gE[k] = C(2) * dq[1] + dq[2];
      dq2[k] = dq[2];
      q2g[k] = q[2] + ldc<C>(a.gB, i);
      wE[k] = E + (a.use_col ? ldc<C>(a.col, s) : C(0));
      dwE[k] = dE + ((a.use_col && a.dcol) ? ldc<C>(a.dcol, s) : C(0));
      lm = fmax(lm, wE[k]);
    }
  }
  const C M = block_max(lm, red);  // its barriers publish X
  const C Ms = M == NI ? C(0) : M;
  C r[CPT], dr[CPT];
  C ls = C(0), lds = C(0);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    r[k] = dr[k] = C(0);
    if (s < S) {
      const int p = t.par[s];
      if (p >= 0) gE[k] += X[p];
      r[k] = xexp2(wE[k] - Ms);
      dr[k] = (C)LN2D * r[k] * dwE[k];
    }
    ls += r[k];
    lds += dr[k];
  }
  const C rowsum = block_sum(ls, red);
  const C drowsum = block_sum(lds, red);
  C anc[CPT], danc[CPT];
  reg_path_sums<CPT>(t, r, anc, EV, red);
  reg_path_sums<CPT>(t, dr, danc, EV, red);
  C u[CPT], du[CPT];
  C lu = C(0), ldu = C(0);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const C denom = rowsum - anc[k];
    const C dden = drowsum - danc[k];
    const bool pos = denom > C(0);
    u[k] = pos ? q2g[k] / denom : C(0);
    du[k] = pos ? (dq2[k] - u[k] * dden) / denom : C(0);
    lu += u[k];
    ldu += du[k];
  }
  const C tot = block_sum(lu, red);
  const C dtot = block_sum(ldu, red);
  C ex[CPT], dex[CPT];
  reg_subtree_sums<CPT>(t, u, ex, EV, red);
  reg_subtree_sums<CPT>(t, du, dex, EV, red);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      const C pv = dr[k] * (tot - ex[k]) + r[k] * (dtot - dex[k]);
      a.oE[base + s] = (T)(gE[k] + pv);
      a.ocol[base + s] = (T)pv;
    }
  }
}

// ---- self-loop J^T and parameter buckets -------------------------------------------------

template <typename T>
struct WsoArgs {
  int S, W, use_col, use_leaf;
  long long ws, cstride;
  const T *Pi, *dPi, *Pb, *dPb, *v, *rowmax;
  const T *DL, *dDL, *Ebar, *dEbar, *E, *dE, *SL1, *dSL1, *SL2, *dSL2, *col;
  const int64_t *item, *leaf_state;
  const T *leaf_logp, *dleaf_logp, *dts, *ddts, *rhs;
  T *out, *aw0, *aw1, *aw2, *aw345, *aw3, *aw4;
};

// One workgroup per wave row w (global row ws + w).  With the sweep's term
// weights w~_k = 2^(t_k - lse), dlse = sum w~_k dt_k, dw~_k = ln2 w~_k (dt_k - dlse),
// the split mixing weight w_L = 2^(lse - Pi_new) and
// dw_L = ln2 w_L (1 - w_L) (dlse - d_dts):
//   d_aw_k = v (dw_L w~_k + w_L dw~_k)
//   d_out  = v d(diag) + dp' (A - sub) + p' (dA - dsub) + [v d(sl_wt)] at the parent,
// u = v w_L w~_2 / denom, A = sum u, sub = subtree sums of u, p' = 2^((col +) Pi - rowmax).
template <typename T, int CPT, typename C = double>
__global__ __launch_bounds__(NT) void wso_kernel(OpsTree t, WsoArgs<T> a) {
  extern __shared__ double smd[];  // raw storage: C values
  const int S = t.S;
  C* Z = reinterpret_cast<C*>(smd);       // child-edge contributions by column
  C* EV = reinterpret_cast<C*>(smd) + S;  // 2S scan buffer
  __shared__ C red[NW];
  const C NI = ninf<C>();
  const int w = blockIdx.x;
  const long long grow = a.ws + w;
  const long long item = a.item[grow];
  const size_t cb = (size_t)(item * a.cstride);
  const size_t lb = (size_t)item * S;
  const size_t rb = (size_t)grow * S;
  const size_t wb = (size_t)w * S;
  const C rm = ldc<C>(a.rowmax, grow);
  const C rms = rm == NI ? C(0) : rm;
  const long long lstate = a.use_leaf ? a.leaf_state[grow] : -1;
  C pp[CPT], dpp[CPT], vv[CPT];
  C lsum = C(0), ldsum = C(0);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    pp[k] = dpp[k] = vv[k] = C(0);
    if (s < S) {
      const C pi = ldc<C>(a.Pi, rb + s);
      pp[k] = xexp2(pi + (a.use_col ? ldc<C>(a.col, s) : C(0)) - rms);
      dpp[k] = (C)LN2D * pp[k] * ldc<C>(a.dPi, rb + s);
      vv[k] = ldc<C>(a.v, wb + s);
      Z[s] = C(0);
    }
    lsum += pp[k];
    ldsum += dpp[k];
  }
  const C rowsum = block_sum(lsum, red);
  const C drowsum = block_sum(ldsum, red);
  C anc[CPT], danc[CPT];
  reg_path_sums<CPT>(t, pp, anc, EV, red);
  reg_path_sums<CPT>(t, dpp, danc, EV, red);
  C dself[CPT], u[CPT], du[CPT];
  C lu = C(0), ldu = C(0);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    dself[k] = u[k] = du[k] = C(0);
    if (s < S) {
      const size_t ci = cb + s;
      const C denom = rowsum - anc[k];
      const C ddenom = drowsum - danc[k];
      const C invd = denom > C(0) ? C(1) / denom : C(0);
      const C pi = ldc<C>(a.Pi, rb + s), dpi = ldc<C>(a.dPi, rb + s);
      const int c1 = t.c1[s], c2 = t.c2[s];
      const C p1 = c1 >= 0 ? ldc<C>(a.Pi, rb + c1) : NI, p2 = c2 >= 0 ? ldc<C>(a.Pi, rb + c2) : NI;
      const C dp1 = c1 >= 0 ? ldc<C>(a.dPi, rb + c1) : C(0), dp2 = c2 >= 0 ? ldc<C>(a.dPi, rb + c2) : C(0);
      const bool hit = lstate == s;
      C tk[6], dtk[6];
      tk[0] = ldc<C>(a.DL, ci) + pi;
      dtk[0] = ldc<C>(a.dDL, ci) + dpi;
      tk[1] = pi + ldc<C>(a.Ebar, ci);
      dtk[1] = dpi + ldc<C>(a.dEbar, ci);
      tk[2] = ldc<C>(a.Pb, rb + s) + ldc<C>(a.E, ci);
      dtk[2] = ldc<C>(a.dPb, rb + s) + ldc<C>(a.dE, ci);
      tk[3] = ldc<C>(a.SL1, ci) + p1;
      dtk[3] = ldc<C>(a.dSL1, ci) + dp1;
      tk[4] = ldc<C>(a.SL2, ci) + p2;
      dtk[4] = ldc<C>(a.dSL2, ci) + dp2;
      tk[5] = hit ? ldc<C>(a.leaf_logp, lb + s) : NI;
      dtk[5] = hit ? ldc<C>(a.dleaf_logp, lb + s) : C(0);
      C m = tk[0];
#pragma unroll
      for (int j = 1; j < 6; ++j) m = fmax(m, tk[j]);
      const C ms = m == NI ? C(0) : m;
      C wk[6], tot = C(0);
#pragma unroll
      for (int j = 0; j < 6; ++j) {
        wk[j] = xexp2(tk[j] - ms);
        tot += wk[j];
      }
      const C inv = tot > C(0) ? C(1) / tot : C(0);
      C dlse = C(0);
#pragma unroll
      for (int j = 0; j < 6; ++j) {
        wk[j] *= inv;
        if (wk[j] != C(0)) dlse += wk[j] * dtk[j];
      }
      C dw[6];
#pragma unroll
      for (int j = 0; j < 6; ++j) dw[j] = wk[j] != C(0) ? (C)LN2D * wk[j] * (dtk[j] - dlse) : C(0);
      C wL = C(1), dwL = C(0);
      if (a.dts) {
        const C dr = ldc<C>(a.dts, wb + s);
        const C dl = tot > C(0) ? xlog2(tot) + m : NI;
        const C pm = fmax(dl, dr);
        const C pms = pm == NI ? C(0) : pm;
        const C pnew = xlog2(xexp2(dl - pms) + xexp2(dr - pms)) + pm;
        wL = dl != NI ? xexp2(dl - pnew) : C(0);
        dwL = (dr != NI && dl != NI) ? (C)LN2D * wL * (C(1) - wL) * (dlse - ldc<C>(a.ddts, wb + s)) : C(0);
      }
      C da[6];
#pragma unroll
      for (int j = 0; j < 6; ++j) da[j] = vv[k] * (dwL * wk[j] + wL * dw[j]);
      a.aw0[wb + s] = (T)da[0];
      a.aw1[wb + s] = (T)da[1];
      a.aw2[wb + s] = (T)da[2];
      a.aw345[wb + s] = (T)(da[3] + da[4] + da[5]);
      a.aw3[wb + s] = (T)da[3];
      a.aw4[wb + s] = (T)da[4];
      if (c1 >= 0) Z[c1] = da[3];
      if (c2 >= 0) Z[c2] = da[4];
      const C pc = wL * wk[2] * invd;
      const C dpc = (dwL * wk[2] + wL * dw[2]) * invd - pc * invd * ddenom;
      u[k] = vv[k] * pc;
      du[k] = vv[k] * dpc;
      dself[k] = da[0] + da[1];
    }
    lu += u[k];
    ldu += du[k];
  }
  const C A = block_sum(lu, red);  // its barriers publish Z
  const C dA = block_sum(ldu, red);
  C sub[CPT], dsub[CPT];
  reg_subtree_sums<CPT>(t, u, sub, EV, red);
  reg_subtree_sums<CPT>(t, du, dsub, EV, red);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      C o = dself[k] + dpp[k] * (A - sub[k]) + pp[k] * (dA - dsub[k]) + Z[s];
      if (a.rhs) o += ldc<C>(a.rhs, rb + s);
      a.out[wb + s] = (T)o;
    }
  }
}

// float32 rows at preorder ownership (thread t owns positions t*CPT + k, as
// the forward and backward row kernels), computed in float32 as the
// reference's Triton kernel computes it: the two root-path sums from one
// pair of preorder / postorder scans, the two subtree sums from one pair of
// published wavefront-local scans, the outputs written back in column order
// through LDS.  Same mathematics as wso_kernel.
template <int CPT>
__global__ __launch_bounds__(NT) void wso_pre_kernel(OpsTree t, WsoArgs<float> a) {
  constexpr int MAXS = NT * CPT;
  constexpr int LD = MAXS + 64;  // [MAXS] is the padding slot, kept at 0
  constexpr int ZERO = MAXS;
  constexpr int SEG = 64 * CPT;  // postorder slots per wavefront
  constexpr float LN2F = 0.69314718055994531f;
  extern __shared__ __align__(16) unsigned char smraw[];
  float* Lr = reinterpret_cast<float*>(smraw);  // 8 rows of LD
  auto row = [&](int j) { return Lr + (size_t)j * LD; };
  __shared__ float wA[2 * NW], wB[2 * NW];
  const int S = t.S;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const float NI = -__builtin_inff();
  const int w = blockIdx.x;
  const long long grow = a.ws + w;
  const long long item = a.item[grow];
  const size_t cb = (size_t)(item * a.cstride);
  const size_t lb = (size_t)item * S;
  const size_t rb = (size_t)grow * S;
  const size_t wb = (size_t)w * S;
  const float rm = a.rowmax[grow];
  const float rms = rm == NI ? 0.0f : rm;
  const long long lstate = a.use_leaf ? a.leaf_state[grow] : -1;
  // Pi, dPi, Pibar, dPibar and v to their preorder positions (rows 0..4)
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) {
      const int p = t.ppos[sc];
      row(0)[p] = a.Pi[rb + sc];
      row(1)[p] = a.dPi[rb + sc];
      row(2)[p] = a.Pb[rb + sc];
      row(3)[p] = a.dPb[rb + sc];
      row(4)[p] = a.v[wb + sc];
    }
  }
  if (tid < 64)
    for (int j = 0; j < 8; ++j) row(j)[MAXS + tid] = 0.0f;
  int colk[CPT], c1p[CPT], c2p[CPT], endm1[CPT], wend[CPT], qp[CPT], nex[CPT];
  bool okp[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = kb::own_pos_c<NT, CPT>(k);
    okp[k] = i < S;
    colk[k] = okp[k] ? t.pcol[i] : 0;
    c1p[k] = okp[k] ? t.pc1[i] : -1;
    c2p[k] = okp[k] ? t.pc2[i] : -1;
    endm1[k] = okp[k] ? t.pend[colk[k]] - 1 : ZERO;
    wend[k] = endm1[k] < ZERO ? endm1[k] / SEG : 0;
    qp[k] = okp[k] ? t.ppost[i] : ZERO;
    nex[k] = okp[k] ? t.pnex[i] : 0;
  }
  {
    // row 7 collects the child-edge terms, written by the parents' owners
    // after the scans below: 0 where a position has no parent
    float zero[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) zero[k] = 0.0f;
    kb::lds_store_own<CPT>(row(7), zero);
  }
  __syncthreads();
  float piv[CPT], dpiv[CPT], pbv[CPT], dpbv[CPT], vv[CPT];
  kb::lds_load_own<CPT>(row(0), piv);
  kb::lds_load_own<CPT>(row(1), dpiv);
  kb::lds_load_own<CPT>(row(2), pbv);
  kb::lds_load_own<CPT>(row(3), dpbv);
  kb::lds_load_own<CPT>(row(4), vv);
  // p' = 2^(Pi + col - rowmax), dp' = ln2 p' dPi and their root-path sums:
  // both preorder scans in registers, rows 5 / 6 hold p' / dp' for the
  // postorder reads, rows 2 / 3 (read above at own positions only) the
  // exclusive postorder scans
  float pp[CPT], dpp[CPT], sa[CPT], sb[CPT], ta = 0.0f, tb = 0.0f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    pp[k] = okp[k] ? exp2f(piv[k] + (a.use_col ? a.col[colk[k]] : 0.0f) - rms) : 0.0f;
    dpp[k] = okp[k] ? LN2F * pp[k] * dpiv[k] : 0.0f;
    ta += pp[k];
    tb += dpp[k];
    sa[k] = ta;
    sb[k] = tb;
  }
  const float wa = kb::wave_scan_incl(ta), wb2 = kb::wave_scan_incl(tb);
  kb::lds_store_own<CPT>(row(5), pp);
  kb::lds_store_own<CPT>(row(6), dpp);
  if (lane == 63) {
    wA[wv] = wa;
    wA[NW + wv] = wb2;
  }
  __syncthreads();
  float anc[CPT], danc[CPT], p1[CPT], p2[CPT], dp1[CPT], dp2[CPT], rowsum, drowsum;
  {
    const float tpa = kb::lds_wave_values<NW>(wA, lane, 0.0f);
    const float tpb = kb::lds_wave_values<NW>(wA + NW, lane, 0.0f);
    float ya[CPT], yb[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      ya[k] = row(5)[qp[k]];
      yb[k] = row(6)[qp[k]];
      p1[k] = c1p[k] >= 0 ? row(0)[c1p[k]] : NI;
      p2[k] = c2p[k] >= 0 ? row(0)[c2p[k]] : NI;
      dp1[k] = c1p[k] >= 0 ? row(1)[c1p[k]] : 0.0f;
      dp2[k] = c2p[k] >= 0 ? row(1)[c2p[k]] : 0.0f;
    }
    const float ipa = kb::wave_scan_first<NW>(tpa), ipb = kb::wave_scan_first<NW>(tpb);
    rowsum = kb::lane_value(ipa, NW - 1);
    drowsum = kb::lane_value(ipb, NW - 1);
    const float offa = kb::lane_value(ipa - tpa, wv) + (wa - ta);
    const float offb = kb::lane_value(ipb - tpb, wv) + (wb2 - tb);
    float qa[CPT], qb[CPT], ua = 0.0f, ub = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      qa[k] = ua;
      qb[k] = ub;
      ua += ya[k];
      ub += yb[k];
    }
    const float xa = kb::wave_scan_incl(ua), xb = kb::wave_scan_incl(ub);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      qa[k] += xa - ua;
      qb[k] += xb - ub;
    }
    kb::lds_store_own<CPT>(row(2), qa);
    kb::lds_store_own<CPT>(row(3), qb);
    if (lane == 63) {
      wB[wv] = xa;
      wB[NW + wv] = xb;
    }
    __syncthreads();
    const float tqa = kb::lds_wave_values<NW>(wB, lane, 0.0f), tqb = kb::lds_wave_values<NW>(wB + NW, lane, 0.0f);
    const float eqa = kb::wave_scan_first<NW>(tqa) - tqa, eqb = kb::wave_scan_first<NW>(tqb) - tqb;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int n = nex[k];
      anc[k] = (sa[k] + offa) - (row(2)[n] + __shfl(eqa, n / SEG, 64));
      danc[k] = (sb[k] + offb) - (row(3)[n] + __shfl(eqb, n / SEG, 64));
    }
  }
  // per position: the second-order bucket terms, the child-edge terms (into
  // row 7 at the child positions) and u = v pc, du = v dpc
  float da[6][CPT], dself[CPT], u[CPT], du[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
#pragma unroll
    for (int j = 0; j < 6; ++j) da[j][k] = 0.0f;
    dself[k] = u[k] = du[k] = 0.0f;
    if (okp[k]) {
      const int s = colk[k];
      const size_t ci = cb + s;
      const float denom = rowsum - anc[k];
      const float ddenom = drowsum - danc[k];
      const float invd = denom > 0.0f ? 1.0f / denom : 0.0f;
      const float pi = piv[k], dpi = dpiv[k];
      const bool hit = lstate == s;
      float tk[6], dtk[6];
      tk[0] = a.DL[ci] + pi;
      dtk[0] = a.dDL[ci] + dpi;
      tk[1] = pi + a.Ebar[ci];
      dtk[1] = dpi + a.dEbar[ci];
      tk[2] = pbv[k] + a.E[ci];
      dtk[2] = dpbv[k] + a.dE[ci];
      tk[3] = a.SL1[ci] + p1[k];
      dtk[3] = a.dSL1[ci] + dp1[k];
      tk[4] = a.SL2[ci] + p2[k];
      dtk[4] = a.dSL2[ci] + dp2[k];
      tk[5] = hit ? a.leaf_logp[lb + s] : NI;
      dtk[5] = hit ? a.dleaf_logp[lb + s] : 0.0f;
      float m = tk[0];
#pragma unroll
      for (int j = 1; j < 6; ++j) m = fmaxf(m, tk[j]);
      const float ms = m == NI ? 0.0f : m;
      float wk[6], tot = 0.0f;
#pragma unroll
      for (int j = 0; j < 6; ++j) {
        wk[j] = exp2f(tk[j] - ms);
        tot += wk[j];
      }
      const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
      float dlse = 0.0f;
#pragma unroll
      for (int j = 0; j < 6; ++j) {
        wk[j] *= inv;
        if (wk[j] != 0.0f) dlse += wk[j] * dtk[j];
      }
      float dw[6];
#pragma unroll
      for (int j = 0; j < 6; ++j) dw[j] = wk[j] != 0.0f ? LN2F * wk[j] * (dtk[j] - dlse) : 0.0f;
      float wL = 1.0f, dwL = 0.0f;
      if (a.dts) {
        const float dr = a.dts[wb + s];
        const float dl = tot > 0.0f ? log2f(tot) + m : NI;
        const float pm = fmaxf(dl, dr);
        const float pms = pm == NI ? 0.0f : pm;
        const float pnew = log2f(exp2f(dl - pms) + exp2f(dr - pms)) + pm;
        wL = dl != NI ? exp2f(dl - pnew) : 0.0f;
        dwL = (dr != NI && dl != NI) ? LN2F * wL * (1.0f - wL) * (dlse - a.ddts[wb + s]) : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 6; ++j) da[j][k] = vv[k] * (dwL * wk[j] + wL * dw[j]);
      if (c1p[k] >= 0) row(7)[c1p[k]] = da[3][k];
      if (c2p[k] >= 0) row(7)[c2p[k]] = da[4][k];
      const float pc = wL * wk[2] * invd;
      const float dpc = (dwL * wk[2] + wL * dw[2]) * invd - pc * invd * ddenom;
      u[k] = vv[k] * pc;
      du[k] = vv[k] * dpc;
      dself[k] = da[0][k] + da[1][k];
    }
  }
  // subtree sums of u and du: wavefront-local scans published in rows 5 / 6
  // (their postorder reads finished before the second barrier above)
  float scu[CPT], scd[CPT];
  kb::local_scan_publish<NT, CPT>(scu, u, row(5), wA);
  kb::local_scan_publish<NT, CPT>(scd, du, row(6), wA + NW);
  __syncthreads();  // also publishes the child-edge terms in row 7
  float pmu[CPT], rsu[CPT], pmd[CPT], rsd[CPT], z[CPT];
  kb::subtree_terms<NT, CPT>(scu, row(5), wA, endm1, wend, pmu, rsu);
  kb::subtree_terms<NT, CPT>(scd, row(6), wA + NW, endm1, wend, pmd, rsd);
  kb::lds_load_own<CPT>(row(7), z);
  // the output row: dself + dp' (A - sub u) + p' (dA - sub du) + the child-edge
  // term from the parent (+ rhs)
  float o[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) o[k] = okp[k] ? dself[k] + dpp[k] * (pmu[k] + rsu[k]) + pp[k] * (pmd[k] + rsd[k]) + z[k] : 0.0f;
  // outputs in column order through rows 0..6, once every thread has read
  // rows 5 / 6 (the subtree terms) and its own entries of row 7
  __syncthreads();
  kb::lds_store_own<CPT>(row(0), o);
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    float x[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) x[k] = j < 5 ? da[j][k] : da[3][k] + da[4][k] + da[5][k];
    kb::lds_store_own<CPT>(row(1 + j), x);
  }
  __syncthreads();
  float* const outs[7] = {a.out, a.aw0, a.aw1, a.aw2, a.aw3, a.aw4, a.aw345};
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) {
      const int p = t.ppos[sc];
      float ov = row(0)[p];
      if (a.rhs) ov += a.rhs[rb + sc];
      outs[0][wb + sc] = ov;
#pragma unroll
      for (int r = 1; r < 7; ++r) outs[r][wb + sc] = row(r)[p];
    }
  }
}

// ---- split-term backward and its Pibar tree VJP --------------------------------------------

template <typename T>
struct DsoArgs {
  int S, by_state, use_col;
  long long N, ws, item_offset, prow, mrow;
  const T *Pi, *dPi, *Pb, *dPb, *v, *lsp, *pD, *pS, *dpD, *dpS, *mt, *dmt, *rowmax, *col;
  const int64_t *sl, *sr, *red, *item, *c1, *c2;
  T *ud, *dud, *side, *colrows, *pDrows, *pSrows, *mtrows;
};

// One workgroup per split n.  w_k = 2^(lsp + d_k - Pi_parent) (0 where Pi_parent = -inf),
// dvd_k = v ln2 w_k (dd_k - dPi_parent); the child rows receive dvd0 + dvd1 (left),
// dvd0 + dvd2 (right) and the speciation terms at the child columns; the Pibar
// cotangents are staged as ud = vd f, dud = dvd f + vd ln2 f (dmt - dPibar) with
// f = 2^(rowmax_child + mt - Pibar).
template <typename T, int CPT>
__global__ __launch_bounds__(NT) void dso_split_kernel(DsoArgs<T> a) {
  // float rows are computed in float32 (hardware exp2), double rows in float64
  using C = typename std::conditional<std::is_same<T, float>::value, float, double>::type;
  const C LN2C = (C)LN2D;
  auto ex2 = [](C x) -> C {
    if constexpr (std::is_same<C, float>::value) return __builtin_amdgcn_exp2f(x);
    else return exp2(x);
  };
  auto ldc = [](const T* p, size_t i) -> C { return (C)p[i]; };
  extern __shared__ double smd[];
  const int S = a.S;
  C* L = reinterpret_cast<C*>(smd);
  C* R = L + S;
  const C NI = -__builtin_inf();
  const long long n = blockIdx.x, N = a.N;
  const long long pw = a.red[n];
  const long long item = a.item[a.item_offset + pw];
  const size_t pb = (size_t)(item * a.prow);
  const size_t mb = (size_t)(item * a.mrow);
  const long long l = a.sl[n], r = a.sr[n];
  const size_t bl = (size_t)l * S, br = (size_t)r * S, bp = (size_t)(a.ws + pw) * S, bv = (size_t)pw * S;
  const C lsp = ldc(a.lsp, n);
  const C rml = ldc(a.rowmax, l), rmr = ldc(a.rowmax, r);
  C d3[CPT], d4[CPT];
  int c1v[CPT], c2v[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    d3[k] = d4[k] = 0;
    c1v[k] = c2v[k] = -1;
    if (s < S) {
      const C d = a.by_state ? ldc(a.pD, pb + s) : ldc(a.pD, pb);
      const C sp = a.by_state ? ldc(a.pS, pb + s) : ldc(a.pS, pb);
      const C dd = a.by_state ? ldc(a.dpD, pb + s) : ldc(a.dpD, pb);
      const C dsp = a.by_state ? ldc(a.dpS, pb + s) : ldc(a.dpS, pb);
      const int c1 = child_at(a.c1, s, S), c2 = child_at(a.c2, s, S);
      c1v[k] = c1;
      c2v[k] = c2;
      const C pl = ldc(a.Pi, bl + s), pr = ldc(a.Pi, br + s);
      const C dpl = ldc(a.dPi, bl + s), dpr = ldc(a.dPi, br + s);
      const C l1 = c1 >= 0 ? ldc(a.Pi, bl + c1) : NI, r1 = c1 >= 0 ? ldc(a.Pi, br + c1) : NI;
      const C l2 = c2 >= 0 ? ldc(a.Pi, bl + c2) : NI, r2 = c2 >= 0 ? ldc(a.Pi, br + c2) : NI;
      const C dl1 = c1 >= 0 ? ldc(a.dPi, bl + c1) : (C)0, dr1 = c1 >= 0 ? ldc(a.dPi, br + c1) : (C)0;
      const C dl2 = c2 >= 0 ? ldc(a.dPi, bl + c2) : (C)0, dr2 = c2 >= 0 ? ldc(a.dPi, br + c2) : (C)0;
      const C pbl = ldc(a.Pb, bl + s), pbr = ldc(a.Pb, br + s);
      const C dpbl = ldc(a.dPb, bl + s), dpbr = ldc(a.dPb, br + s);
      const C dk[5] = {d + pl + pr, pl + pbr, pr + pbl, sp + l1 + r2, sp + r1 + l2};
      const C ddk[5] = {dd + dpl + dpr, dpl + dpbr, dpr + dpbl, dsp + dl1 + dr2, dsp + dr1 + dl2};
      const C pp = ldc(a.Pi, bp + s), dpp = ldc(a.dPi, bp + s);
      const C vv = ldc(a.v, bv + s);
      C wk[5], dv[5];
#pragma unroll
      for (int j = 0; j < 5; ++j) {
        wk[j] = pp != NI ? ex2(lsp + dk[j] - pp) : (C)0;
        dv[j] = wk[j] != (C)0 ? vv * LN2C * wk[j] * (ddk[j] - dpp) : (C)0;
      }
      L[s] = dv[0] + dv[1];
      R[s] = dv[0] + dv[2];
      d3[k] = dv[3];
      d4[k] = dv[4];
      const C mt = ldc(a.mt, mb + s), dmt = ldc(a.dmt, mb + s);
      const C fl = pbl != NI ? ex2(rml + mt - pbl) : (C)0;
      const C fr = pbr != NI ? ex2(rmr + mt - pbr) : (C)0;
      const C vd1 = vv * wk[1], vd2 = vv * wk[2];
      const size_t ol = (size_t)n * S + s, orr = (size_t)(N + n) * S + s;
      a.ud[ol] = (T)(vd2 * fl);
      a.ud[orr] = (T)(vd1 * fr);
      a.dud[ol] = (T)(dv[2] * fl + (fl != (C)0 ? vd2 * LN2C * fl * (dmt - dpbl) : (C)0));
      a.dud[orr] = (T)(dv[1] * fr + (fr != (C)0 ? vd1 * LN2C * fr * (dmt - dpbr) : (C)0));
      a.pDrows[(size_t)n * S + s] = (T)dv[0];
      a.pSrows[(size_t)n * S + s] = (T)(dv[3] + dv[4]);
      a.mtrows[(size_t)n * S + s] = (T)(dv[1] + dv[2]);
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    if (c1v[k] >= 0) {
      L[c1v[k]] += d3[k];
      R[c1v[k]] += d4[k];
    }
    if (c2v[k] >= 0) {
      R[c2v[k]] += d3[k];
      L[c2v[k]] += d4[k];
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      a.side[(size_t)n * S + s] = (T)L[s];
      a.side[(size_t)(N + n) * S + s] = (T)R[s];
    }
  }
}

// One workgroup per split side i (i < N: left child sl[i], else right child
// sr[i - N]): contrib = dp' (A - sub) + p' (dA - dsub) over the staged ud / dud,
// p' = 2^((col +) Pi_child - rowmax_child), dp' = ln2 p' dPi_child; added to
// the side row and written as the side's column-gradient row.
template <typename T, int CPT>
__global__ __launch_bounds__(NT) void dso_tree_kernel(OpsTree t, DsoArgs<T> a) {
  extern __shared__ double smd[];
  double* buf = smd;
  __shared__ double red[NW];
  const int S = a.S;
  const double NI = -__builtin_inf();
  const long long i = blockIdx.x, N = a.N;
  const long long child = i < N ? a.sl[i] : a.sr[i - N];
  const size_t rb = (size_t)i * S, cbase = (size_t)child * S;
  const double rm = ld(a.rowmax, child);
  const double rms = rm == NI ? 0.0 : rm;
  double x[CPT], dx[CPT];
  double lA = 0.0, ldA = 0.0;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    x[k] = s < S ? ld(a.ud, rb + s) : 0.0;
    dx[k] = s < S ? ld(a.dud, rb + s) : 0.0;
    lA += x[k];
    ldA += dx[k];
  }
  const double A = block_sum(lA, red);
  const double dA = block_sum(ldA, red);
  double sub[CPT], dsub[CPT];
  reg_subtree_sums<CPT>(t, x, sub, buf, red);
  reg_subtree_sums<CPT>(t, dx, dsub, buf, red);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      const double pi = ld(a.Pi, cbase + s);
      const double pp = pi != NI ? exp2(pi + (a.use_col ? ld(a.col, s) : 0.0) - rms) : 0.0;
      const double c = LN2D * pp * ld(a.dPi, cbase + s) * (A - sub[k]) + pp * (dA - dsub[k]);
      a.side[rb + s] = (T)(ld(a.side, rb + s) + c);
      a.colrows[rb + s] = (T)c;
    }
  }
}

// dso_tree_kernel for float32 rows at preorder ownership (thread t owns the
// contiguous positions t*CPT + k): ud / dud and the child's Pi / dPi rows are
// staged to their preorder positions, both subtree complements A - sub come
// from wavefront-local scans published behind one barrier, and the outputs go
// back to column order through LDS.  Same terms as dso_tree_kernel, in
// float32 with the hardware exp2.
template <int CPT>
__global__ __launch_bounds__(NT) void dso_tree_pre_kernel(OpsTree t, DsoArgs<float> a) {
  constexpr int MAXS = NT * CPT;
  constexpr int LD = MAXS + 64;  // [MAXS] is the padding slot, kept at 0
  constexpr int ZERO = MAXS;
  constexpr int SEG = 64 * CPT;  // positions per wavefront
  constexpr float LN2F = 0.69314718055994531f;
  extern __shared__ __align__(16) unsigned char smraw[];
  float* Lr = reinterpret_cast<float*>(smraw);  // rows: ud, dud (then their scans), Pi (then the output), dPi
  auto row = [&](int j) { return Lr + (size_t)j * LD; };
  __shared__ float wA[NW], wB[NW];
  const int S = t.S;
  const int tid = threadIdx.x;
  const float NI = -__builtin_inff();
  const long long i = blockIdx.x, N = a.N;
  const long long child = i < N ? a.sl[i] : a.sr[i - N];
  const size_t rb = (size_t)i * S, cbase = (size_t)child * S;
  const float rm = a.rowmax[child];
  const float rms = rm == NI ? 0.0f : rm;
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) {
      const int p = t.ppos[sc];
      row(0)[p] = a.ud[rb + sc];
      row(1)[p] = a.dud[rb + sc];
      row(2)[p] = a.Pi[cbase + sc];
      row(3)[p] = a.dPi[cbase + sc];
    }
  }
  if (tid < 64)
    for (int j = 0; j < 4; ++j) row(j)[MAXS + tid] = 0.0f;
  int colk[CPT], endm1[CPT], wend[CPT];
  bool okp[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int q = kb::own_pos_c<NT, CPT>(k);
    okp[k] = q < S;
    colk[k] = okp[k] ? t.pcol[q] : 0;
    endm1[k] = okp[k] ? t.pend[colk[k]] - 1 : ZERO;
    wend[k] = endm1[k] < ZERO ? endm1[k] / SEG : 0;
  }
  __syncthreads();
  float x[CPT], dx[CPT], pi[CPT], dpi[CPT];
  kb::lds_load_own<CPT>(row(0), x);
  kb::lds_load_own<CPT>(row(1), dx);
  kb::lds_load_own<CPT>(row(2), pi);
  kb::lds_load_own<CPT>(row(3), dpi);
#pragma unroll
  for (int k = 0; k < CPT; ++k)
    if (!okp[k]) x[k] = dx[k] = 0.0f;  // positions past S were not written: out of the scans
  float sx[CPT], sdx[CPT];
  kb::local_scan_publish<NT, CPT>(sx, x, row(0), wA);
  kb::local_scan_publish<NT, CPT>(sdx, dx, row(1), wB);
  __syncthreads();
  float pm1[CPT], rest[CPT], dpm1[CPT], drest[CPT];
  kb::subtree_terms<NT, CPT>(sx, row(0), wA, endm1, wend, pm1, rest);
  kb::subtree_terms<NT, CPT>(sdx, row(1), wB, endm1, wend, dpm1, drest);
  float c[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    c[k] = 0.0f;
    if (okp[k]) {
      const float pp = pi[k] != NI ? __builtin_amdgcn_exp2f(pi[k] + (a.use_col ? a.col[colk[k]] : 0.0f) - rms) : 0.0f;
      c[k] = LN2F * pp * dpi[k] * (pm1[k] + rest[k]) + pp * (dpm1[k] + drest[k]);
    }
  }
  kb::lds_store_own<CPT>(row(2), c);  // row 2 was read only at own positions
  __syncthreads();
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int sc = tid + j * NT;
    if (sc < S) {
      const float v = row(2)[t.ppos[sc]];
      a.side[rb + sc] += v;
      a.colrows[rb + sc] = v;
    }
  }
}

}  // namespace kbo

using namespace kbo_host;

namespace {

// float32 rows of up to 4096 states run the preorder-ownership kernel, the
// others the generic one (float64 arithmetic, float32 for float32 rows too
// long for three float64 LDS rows)
template <typename T, int CPT>
int launch_wso(const kbo::OpsTree& t, const kbo::WsoArgs<T>& a, int W, bool f32, size_t lds, hipStream_t st) {
  if constexpr (std::is_same_v<T, float> && CPT <= 4) {  // (eight LDS rows: up to 4096 positions)
    const size_t lds_pre = (size_t)8 * (kbo::NT * CPT + 64) * sizeof(float);
    auto k = kbo::wso_pre_kernel<CPT>;
    if (int rc = set_lds(k, lds_pre)) return rc;
    hipLaunchKernelGGL(k, dim3(W), dim3(kbo::NT), lds_pre, st, t, a);
    return 0;
  }
  if constexpr (std::is_same_v<T, float> && CPT == 8) {
    if (f32) {  // rows too long for three float64 LDS rows
      auto k = kbo::wso_kernel<T, CPT, float>;
      if (int rc = set_lds(k, lds)) return rc;
      hipLaunchKernelGGL(k, dim3(W), dim3(kbo::NT), lds, st, t, a);
      return 0;
    }
  }
  if (f32) return kb::set_error(KB_ERR_ARG, "S=%d: no float32 wso_kernel for %d positions per thread", a.S, CPT);
  auto k = kbo::wso_kernel<T, CPT>;
  if (int rc = set_lds(k, lds)) return rc;
  hipLaunchKernelGGL(k, dim3(W), dim3(kbo::NT), lds, st, t, a);
  return 0;
}

template <typename T, int CPT>
int launch_eso(const kbo::OpsTree& t, const kbo::EsoArgs<T>& a, bool f32, size_t lds, hipStream_t st) {
  if constexpr (std::is_same_v<T, float> && CPT == 8) {
    if (f32) {  // rows too long for three float64 LDS rows
      auto k = kbo::eso_kernel<T, CPT, float>;
      if (int rc = set_lds(k, lds)) return rc;
      hipLaunchKernelGGL(k, dim3(a.G), dim3(kbo::NT), lds, st, t, a);
      return 0;
    }
  }
  if (f32) return kb::set_error(KB_ERR_ARG, "S=%d: no float32 eso_kernel for %d positions per thread", a.S, CPT);
  auto k = kbo::eso_kernel<T, CPT>;
  if (int rc = set_lds(k, lds)) return rc;
  hipLaunchKernelGGL(k, dim3(a.G), dim3(kbo::NT), lds, st, t, a);
  return 0;
}

// float32 rows: the preorder-ownership tree kernel; the others the float64 one
template <typename T, int CPT>
int launch_dso_tree(const kbo::OpsTree& t, const kbo::DsoArgs<T>& a, size_t lds, hipStream_t st) {
  const dim3 grid((unsigned)(2 * a.N));
  if constexpr (std::is_same_v<T, float>) {
    const size_t lds_pre = (size_t)4 * (kbo::NT * CPT + 64) * sizeof(float);
    auto k = kbo::dso_tree_pre_kernel<CPT>;
    if (int rc = set_lds(k, lds_pre)) return rc;
    hipLaunchKernelGGL(k, grid, dim3(kbo::NT), lds_pre, st, t, a);
    return 0;
  }
  auto k = kbo::dso_tree_kernel<T, CPT>;
  if (int rc = set_lds(k, lds)) return rc;
  hipLaunchKernelGGL(k, grid, dim3(kbo::NT), lds, st, t, a);
  return 0;
}

}  // namespace

extern "C" {

int kb_estep_backward_so(const kb_tree* tr, const kb_estep_so_io* io, void* stream) {
  if (!tr || !io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->G < 0) return kb::set_error(KB_ERR_ARG, "G must be non-negative");
  if (io->G == 0) return 0;
  const int S = tr->S;
  size_t lds;
  bool f32;
  if (int rc = three_row_lds(S, io->dtype, &lds, &f32)) return rc;
  const kbo::OpsTree t = tr->dev();
  KBO_DISPATCH(io->dtype, S, {
    kbo::EsoArgs<T> a{io->G, S, io->use_col_weights,
                      (const T*)io->E, (const T*)io->E_new, (const T*)io->E_s1, (const T*)io->E_s2,
                      (const T*)io->Ebar, (const T*)io->log_pS, (const T*)io->log_pD, (const T*)io->log_pL,
                      (const T*)io->col_log_probs, (const T*)io->g_new, (const T*)io->g_ebar,
                      (const T*)io->dE, (const T*)io->dE_new, (const T*)io->dE_s1, (const T*)io->dE_s2,
                      (const T*)io->dEbar, (const T*)io->dlog_pS, (const T*)io->dlog_pD, (const T*)io->dlog_pL,
                      (const T*)io->dcol, (T*)io->d_grad_E, (T*)io->d_grad_pS, (T*)io->d_grad_pD,
                      (T*)io->d_grad_pL, (T*)io->d_grad_mc, (T*)io->col_rows};
    if (int rc = launch_eso<T, CPT>(t, a, f32, lds, st_of(stream))) return rc;
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_wave_backward_so(const kb_tree* tr, const kb_wave_so_io* io, void* stream) {
  if (!tr || !io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->S != tr->S) return kb::set_error(KB_ERR_ARG, "S=%d does not match the tree (%d)", io->S, tr->S);
  if (io->W < 0) return kb::set_error(KB_ERR_ARG, "W must be non-negative");
  if ((io->dts == nullptr) != (io->d_dts == nullptr))
    return kb::set_error(KB_ERR_ARG, "dts and d_dts must be given together");
  if (io->W == 0) return 0;
  const int S = tr->S;
  size_t lds;
  bool f32;
  if (int rc = three_row_lds(S, io->dtype, &lds, &f32)) return rc;
  const kbo::OpsTree t = tr->dev();
  KBO_DISPATCH(io->dtype, S, {
    kbo::WsoArgs<T> a{S, io->W, io->use_col_weights, io->use_leaf_index, io->ws, io->const_stride,
                      (const T*)io->Pi, (const T*)io->dPi, (const T*)io->Pibar, (const T*)io->dPibar,
                      (const T*)io->v, (const T*)io->pibar_row_max, (const T*)io->DL, (const T*)io->dDL,
                      (const T*)io->Ebar, (const T*)io->dEbar, (const T*)io->E, (const T*)io->dE,
                      (const T*)io->SL1, (const T*)io->dSL1, (const T*)io->SL2, (const T*)io->dSL2,
                      (const T*)io->col_log_probs, io->item_idx, io->leaf_state, (const T*)io->leaf_logp,
                      (const T*)io->dleaf_logp, (const T*)io->dts, (const T*)io->d_dts, (const T*)io->d_rhs,
                      (T*)io->d_out, (T*)io->d_aw0, (T*)io->d_aw1, (T*)io->d_aw2, (T*)io->d_aw345,
                      (T*)io->d_aw3, (T*)io->d_aw4};
    if (int rc = launch_wso<T, CPT>(t, a, io->W, f32, lds, st_of(stream))) return rc;
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

int kb_dts_backward_so(const kb_tree* tr, const kb_dts_so_io* io, void* stream) {
  if (!tr || !io) return kb::set_error(KB_ERR_ARG, "null argument");
  if (int rc = dtype_ok(io->dtype)) return rc;
  if (io->S != tr->S) return kb::set_error(KB_ERR_ARG, "S=%d does not match the tree (%d)", io->S, tr->S);
  if (io->N < 0) return kb::set_error(KB_ERR_ARG, "N must be non-negative");
  if (io->N == 0) return 0;
  if (io->N > (1LL << 30)) return kb::set_error(KB_ERR_ARG, "N=%lld too large", (long long)io->N);
  const int S = tr->S;
  const size_t lds2 = (size_t)2 * S * sizeof(double), lds1 = (size_t)S * sizeof(double);
  if (int rc = check_lds(lds2, S, KB_F64)) return rc;
  const kbo::OpsTree t = tr->dev();
  KBO_DISPATCH(io->dtype, S, {
    kbo::DsoArgs<T> a{S, io->param_by_state, io->use_col_weights, io->N, io->ws, io->item_offset,
                      io->param_row_stride, io->mt_row_stride,
                      (const T*)io->Pi, (const T*)io->dPi, (const T*)io->Pibar, (const T*)io->dPibar,
                      (const T*)io->v, (const T*)io->log_split_probs, (const T*)io->log_pD, (const T*)io->log_pS,
                      (const T*)io->dlog_pD, (const T*)io->dlog_pS, (const T*)io->mt, (const T*)io->dmt,
                      (const T*)io->pibar_row_max, (const T*)io->col_log_probs,
                      io->sl, io->sr, io->reduce_idx, io->item_idx, io->node_child1, io->node_child2,
                      (T*)io->ud, (T*)io->dud, (T*)io->side_rows, (T*)io->col_rows, (T*)io->pD_rows,
                      (T*)io->pS_rows, (T*)io->mt_rows};
    if (int rc = set_lds(kbo::dso_split_kernel<T, CPT>, lds2)) return rc;
    hipLaunchKernelGGL((kbo::dso_split_kernel<T, CPT>), dim3((unsigned)io->N), dim3(kbo::NT), lds2,
                       st_of(stream), a);
    if (int rc = launch_dso_tree<T, CPT>(t, a, lds1, st_of(stream))) return rc;
  });
  KBO_HIP(hipGetLastError());
  return 0;
}

}  // extern "C"
