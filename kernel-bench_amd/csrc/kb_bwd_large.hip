// Backward row kernel for species trees of 2049 to 8192 nodes.
//
// Same per-row mathematics as bwd_row_kernel (kb_bwd.hip; reference
// kbench/api/_implicit_grad.py:97-370 driving pristine wave_backward.py):
// adjoint gather or root seed, active mask, split term at Pi*, J^T
// coefficients, Neumann series, self-loop column gradient and parameter
// buckets, split adjoints into the children's staging rows.
//
// At these sizes a row needs 1024 threads owning 4 or 8 preorder positions
// each, and 16 wavefronts per workgroup leave 128 VGPRs per thread.  The
// general kernel keeps per-position tables, six coefficient rows and eight
// bucket rows in registers across the whole row and spills hundreds of
// registers there.  This kernel keeps across phases only what the Neumann
// series needs:
//  * per-position tables (children, parent, subtree end, postorder slot) are
//    read from memory in the phase that uses them (L2-resident, 32 KB each);
//  * per-position constants are read from memory where they are used;
//  * the J^T coefficients q_0..q_5 are recomputed after the Neumann series
//    from Pi*, Pibar* and the split term (same code, same values) instead of
//    being held through it;
//  * the gradient buckets are added into this workgroup's bucket slot in
//    memory after every row (each thread updates only its own positions, in
//    row order, so the sums keep a fixed order).
#include "kb_device.hpp"
#include "kb_kernels.hpp"
#include "kb_rowops.hpp"

namespace kb {

namespace {

// the per-position constants the coefficients read
struct CoefK {
  float DL, Ebar, E, SL1, SL2, pS;
};

// q_0..q_5 of own position i: the self-loop terms' shares of the row's
// log-sum (wave_backward.py:264-416), with the split mixing weight folded into
// the normaliser, q_j = e_j / (sum_j e_j + 2^(dts - m)).
struct Coef6 {
  float q[6];
};

__device__ __forceinline__ Coef6 coef_at(const CoefK& K, float piv, float pbv, float dts, float pc1, float pc2,
                                         bool leaf_row, bool is_leaf_pos) {
  const float t0 = K.DL + piv;
  const float t1 = piv + K.Ebar;
  const float t2 = pbv + K.E;
  const float t3 = K.SL1 + pc1;
  const float t4 = K.SL2 + pc2;
  const float t5 = is_leaf_pos ? K.pS : KB_NEG_INF;
  const float m = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), fmaxf(t4, t5));
  const float msf = fsafe(m);
  Coef6 c;
  c.q[0] = exp2_hw(t0 - msf);
  c.q[1] = exp2_hw(t1 - msf);
  c.q[2] = exp2_hw(t2 - msf);
  c.q[3] = exp2_hw(t3 - msf);
  c.q[4] = exp2_hw(t4 - msf);
  c.q[5] = exp2_hw(t5 - msf);
  const float sum = c.q[0] + c.q[1] + c.q[2] + c.q[3] + c.q[4] + c.q[5];
  const float den = sum + (leaf_row ? 0.0f : exp2_hw(dts - msf));
  const float inv = sum > 0.0f ? rcp_hw(den) : 0.0f;
#pragma unroll
  for (int j = 0; j < 6; ++j) c.q[j] *= inv;
  return c;
}

}  // namespace

template <int N>
__device__ __forceinline__ void vld(const float* p, float (&x)[N]) {
#pragma unroll
  for (int k = 0; k < N; k += 4) {
    const float4 q = *reinterpret_cast<const float4*>(p + k);
    x[k] = q.x;
    x[k + 1] = q.y;
    x[k + 2] = q.z;
    x[k + 3] = q.w;
  }
}

template <int N>
__device__ __forceinline__ void vst(float* p, const float (&x)[N]) {
#pragma unroll
  for (int k = 0; k < N; k += 4) *reinterpret_cast<float4*>(p + k) = make_float4(x[k], x[k + 1], x[k + 2], x[k + 3]);
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float f4(const float4& v, int j) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; }
// *p = b + x (four floats)
__device__ __forceinline__ void st4_add(float* p, float4 b, const float (&x)[4]) {
  b.x += x[0];
  b.y += x[1];
  b.z += x[2];
  b.w += x[3];
  *reinterpret_cast<float4*>(p) = b;
}

// NT threads (1024, or 512 for rows of at most 2048 states) own CPT positions
// each; at most 128 VGPRs, so 16 wavefronts per CU are resident (two
// workgroups of 512).
// EARLY: the Neumann series may stop early (P.rtol > 0), as in bwd_row_kernel
template <int NT, int CPT, bool WEIGHTED, bool EARLY>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4)))
void bwd_row_large_kernel(BwdParams P, int first, int n_rows, int poff) {
  constexpr int MAXS = NT * CPT;
  constexpr int LD = MAXS + 64;  // [MAXS] is the padding slot, kept at 0
  constexpr int NW = NT / 64;
  constexpr int ZERO = MAXS;
  constexpr int SEGSH = CPT == 4 ? 8 : 9;  // log2 of the positions per wavefront
  constexpr int NG = CPT / 4;              // groups of four own positions
  static_assert(CPT == 4 || CPT == 8, "4 or 8 positions per thread");
  static_assert(NT == 512 || NT == 1024, "512 or 1024 threads");
  __shared__ float L[4 * LD];
  __shared__ float wA[2 * NW], wB[2 * NW];
  __shared__ float wMk[NW];
  float* R0 = L;
  float* R1 = L + LD;
  float* R2 = L + 2 * LD;
  float* R3 = L + 3 * LD;

  const PreDev& T = P.pre;
  const int S = P.S;
  const int tid = threadIdx.x;
  const int wv = tid >> 6, lane = tid & 63;
  if (tid < 64) {
    R0[MAXS + tid] = 0.0f;
    R1[MAXS + tid] = 0.0f;
    R2[MAXS + tid] = 0.0f;
    R3[MAXS + tid] = 0.0f;
  }
  // this workgroup's slot (KB_LARGE_SLOT_ROWS rows of MAXS floats, preorder
  // positions): the eight bucket rows, then the current row's split term, Pi*
  // and Pibar*.  srow(j) is this thread's first own position of row j.
  float* const slot = P.contrib + (size_t)(poff + (int)blockIdx.x) * KB_LARGE_SLOT_ROWS * MAXS;
  int ep = 0;  // epoch of the current phase (see fresh)
  auto srow = [&](int j) {
    return reinterpret_cast<float*>(reinterpret_cast<char*>(fresh(slot + (size_t)j * MAXS, ep)) +
                                    (unsigned)(tid * CPT) * 4u);
  };
  enum { SL_DTS = 8, SL_PI = 9, SL_PIBAR = 10 };
  // own position k; with 8 positions per thread recomputed where it is used
  // (the positions and the LDS addresses derived from them would otherwise be
  // held across the row loop)
  auto pos = [&](int k) {
    int b = tid * CPT;
    if constexpr (CPT > 4) asm("; %1" : "+v"(b) : "s"(ep));
    return b + k;
  };
  // a global row in column order -> LDS at preorder positions (coalesced reads)
  auto stage = [&](float* dst, const float* src) {
    int sp[CPT];
    float x[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int s = tid + j * NT;
      sp[j] = s < S ? ldg(fresh(T.pre, ep), s) : -1;
      x[j] = s < S ? ldg(fresh(src, ep), s) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j)
      if (sp[j] >= 0) dst[sp[j]] = x[j];
  };
  auto field = [](int rec, int f) { return __builtin_amdgcn_readlane(rec, f); };
  // row j of the owner-major tables / constants at own position k (one
  // contiguous read per wavefront)
  auto omi = [&](int j, int k) { return ldg(fresh(P.om_tab + (size_t)j * MAXS + k * NT, ep), tid); };
  auto omf = [&](int j, int k) { return ldg(fresh(P.om_const + (size_t)j * MAXS + k * NT, ep), tid); };
  auto coef_k = [&](int k) {
    return CoefK{omf(OMC_DL, k), omf(OMC_EBAR, k), omf(OMC_E, k), omf(OMC_SL1, k), omf(OMC_SL2, k), omf(OMC_PS, k)};
  };
  // subtree-sum offsets of a scan published by local_scan_publish: the block
  // total A, this wavefront's offset, and lane x < NW holding wavefront x's
  auto scan_offsets = [&](const float* wt, float& A, float& woff, float& wexcl) {
    const float wtot = lds_wave_values<NW>(wt, lane, 0.0f);
    const float wincl = wave_scan_first<NW>(wtot);
    wexcl = wincl - wtot;
    A = lane_value(wincl, NW - 1);
    woff = lane_value(wexcl, wv);
  };

  for (int rr = blockIdx.x; rr < n_rows; rr += gridDim.x) {
    __syncthreads();  // LDS of the previous row is no longer read
    ep = rr * 16 + 1;
    const int cm = P.class_mode;
    const int rec = cm ? 0 : P.bslot[(size_t)KB_BREC * (first + rr) + (tid & (KB_BREC - 1))];
    const int f_row = field(rec, BR_ROW), f_leaf = field(rec, BR_LEAF), f_sb = field(rec, BR_SB);
    const int f_se = field(rec, BR_SE), f_fam = field(rec, BR_FAM), f_s0 = field(rec, BR_S0);
    const int f_s1 = field(rec, BR_S1), f_lpos = field(rec, BR_LPOS), f_rep = field(rec, BR_REP);
    const int row = cm ? P.cls_rows[P.cls_ptr[rr]] : f_row;
    const bool leaf_row = (cm ? P.row_kind[row] : f_leaf) != 0;
    const int sb = cm ? P.split_ptr[row] : f_sb, se = cm ? P.split_ptr[row + 1] : f_se;
    const int fam = cm ? -1 : f_fam;
    const size_t rb = (size_t)row * S;

    // ---- 1. adjoint: the class's summed adjoint, the root seed (below), or the
    // fixed-order gather of the live staging rows of the row's child sides.
    // The row's loads are issued together: Pi* / Pibar* (columns tid + j*NT,
    // to LDS below), the first two child sides' flags and staging rows (added
    // when live), and the stored split term.
    float nPi[CPT], nPb[CPT];
    int spre[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int s = tid + j * NT;
      spre[j] = s < S ? ldg(fresh(T.pre, ep), s) : -1;
      nPi[j] = s < S ? ldg(fresh(P.pi + rb, ep), s) : 0.0f;
      nPb[j] = s < S ? ldg(fresh(P.pibar + rb, ep), s) : 0.0f;
    }
    float rhs[CPT], dts[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) dts[k] = KB_NEG_INF;
    if (!leaf_row && P.dts_in) {
      const float* src = P.dts_in + (size_t)(cm ? P.rep_of[row] : f_rep) * S;
#pragma unroll
      for (int k = 0; k < CPT; ++k)
        if (pos(k) < S) dts[k] = ldg(fresh(src, ep), pos(k));
    }
    bool any_active = false;
    float row_amax = 0.0f;  // max |adjoint| of the row
    if (cm) {
      any_active = P.cls_active[rr] != 0;
      const float* src = P.rhsc + (size_t)rr * S;
#pragma unroll
      for (int k = 0; k < CPT; ++k) rhs[k] = pos(k) < S ? ldg(fresh(src, ep), pos(k)) : 0.0f;
    } else {
      const int s1 = f_s1 < 0 ? -1 : (f_s1 & ((1 << 30) - 1));
      const bool on0 = f_s0 >= 0 && P.split_on[f_s0 >> 1];
      const bool on1 = s1 >= 0 && P.split_on[s1 >> 1];
      const float* st0 = P.staging + (size_t)(f_s0 >= 0 ? f_s0 : 0) * kb_stage_ld(S);
      const float* st1 = P.staging + (size_t)(s1 >= 0 ? s1 : 0) * kb_stage_ld(S);
      float a0[CPT], a1[CPT];
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const bool ok = pos(k) < S;
        a0[k] = ok && f_s0 >= 0 ? ldg(fresh(st0, ep), pos(k)) : 0.0f;
        a1[k] = ok && s1 >= 0 ? ldg(fresh(st1, ep), pos(k)) : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        rhs[k] = 0.0f;
        if (on0) rhs[k] += a0[k];
        if (on1) rhs[k] += a1[k];
      }
      const int n2 = (f_s1 >= 0 && (f_s1 >> 30) != 0) ? P.child_ptr[row + 1] - P.child_ptr[row] - 2 : 0;
      for (int j = 0; j < n2; ++j) {
        const int side = P.child_in[P.child_ptr[row] + 2 + j];
        if (!P.split_on[side >> 1]) continue;
        const float* st = P.staging + (size_t)side * kb_stage_ld(S);
#pragma unroll
        for (int k = 0; k < CPT; ++k)
          if (pos(k) < S) rhs[k] += ldg(fresh(st, ep), pos(k));
      }
    }
    const bool mask_early = !cm && fam < 0;
    // (class rows publish them too when the Neumann series may stop early: its
    // threshold is relative to the row's largest adjoint entry)
    if (mask_early || (EARLY && cm)) {
      float am = 0.0f;
#pragma unroll
      for (int k = 0; k < CPT; ++k) am = fmaxf(am, fabsf(rhs[k]));
      const float wm = wave_reduce_max(am);
      if (lane == 0) wMk[wv] = wm;
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j)
      if (spre[j] >= 0) {
        R0[spre[j]] = nPi[j];
        R1[spre[j]] = nPb[j];
      }
    __syncthreads();
    float piv[CPT];
    lds_load_own<CPT>(R0, piv);
#pragma unroll
    for (int k = 0; k < CPT; ++k)
      if (pos(k) >= S) piv[k] = KB_NEG_INF;
    if (EARLY && cm) {
#pragma unroll
      for (int w = 0; w < NW; ++w) row_amax = fmaxf(row_amax, wMk[w]);
    }
    if (!cm) {
      if (fam >= 0) {
        // logsumexp2 (logspace.py:11-16) and _safe_exp2_ratio (_implicit_grad.py:21-25)
        float lm = KB_NEG_INF;
#pragma unroll
        for (int k = 0; k < CPT; ++k) lm = fmaxf(lm, piv[k]);
        const float rmax = block_max1<NT>(lm, wA);
        const float rmx = fsafe(rmax);
        float ls = 0.0f;
#pragma unroll
        for (int k = 0; k < CPT; ++k) ls += pos(k) < S ? exp2f(piv[k] - rmx) : 0.0f;
        const float tot = block_sum1<NT>(ls, wB);
        const float lse = (tot > 0.0f ? log2f(tot) : KB_NEG_INF) + rmax;
        const float lses = fsafe(lse);
#pragma unroll
        for (int k = 0; k < CPT; ++k) rhs[k] = (piv[k] == KB_NEG_INF) ? 0.0f : -exp2f(piv[k] - lses);
      }
      // ---- 2. active mask (the reference's rule, wave_backward.py:150-163)
      float amax;
      if (mask_early) {
        amax = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) amax = fmaxf(amax, wMk[w]);
      } else {
        float am = 0.0f;
#pragma unroll
        for (int k = 0; k < CPT; ++k) am = fmaxf(am, fabsf(rhs[k]));
        amax = block_max1<NT>(am, wA);
      }
      any_active = P.use_pruning ? (amax >= P.thr) : (amax > P.thr);
      if (tid == 0) P.mask[row] = any_active ? 1 : 0;
      row_amax = amax;
    }
    if (!any_active) {
      for (int i = sb + tid; i < se; i += NT) P.split_on[i] = 0;
      continue;
    }
    const float rms = fsafe(P.rowmax[row]);
    const int lpos = cm ? (leaf_row ? T.pre[P.leaf_state[row]] : -1) : f_lpos;
    // Pibar* at the own positions (each thread reads its own positions only,
    // before any thread restages R1); Pi* and Pibar* kept in the slot for the
    // phases after the Neumann series
    float pbv[CPT];
    lds_load_own<CPT>(R1, pbv);
#pragma unroll
    for (int k = 0; k < CPT; ++k)
      if (pos(k) >= S) pbv[k] = KB_NEG_INF;
    vst<CPT>(srow(SL_PI), piv);
    vst<CPT>(srow(SL_PIBAR), pbv);
    // the reductions above reused scratch, and the split term below restages
    // R0..R3 when it is not stored
    if (fam >= 0 || (!leaf_row && !P.dts_in)) __syncthreads();

    // ---- 3. split term at Pi* (split rows)
    // (a stored split term was loaded with the row)
    ep = rr * 16 + 3;
    if (!leaf_row && !P.dts_in) {
      float acc[CPT];
#pragma unroll
      for (int k = 0; k < CPT; ++k) acc[k] = 0.0f;
      for (int si = sb; si < se; ++si) {
        const size_t l = (size_t)P.split_l[si] * S, r = (size_t)P.split_r[si] * S;
        const float lsp = P.split_lsp[si];
        stage(R0, P.pi + l);
        stage(R1, P.pi + r);
        stage(R2, P.pibar + l);
        stage(R3, P.pibar + r);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
          const int i = pos(k);
          if (i < S) {
            const int c1 = omi(OMT_C1, k), c2 = omi(OMT_C2, k);
            const float pl = R0[i], pr = R1[i];
            const float l1 = c1 >= 0 ? R0[c1] : KB_NEG_INF, r1 = c1 >= 0 ? R1[c1] : KB_NEG_INF;
            const float l2 = c2 >= 0 ? R0[c2] : KB_NEG_INF, r2 = c2 >= 0 ? R1[c2] : KB_NEG_INF;
            const float t0 = lsp + omf(OMC_PD, k) + pl + pr;
            const float t1 = lsp + pl + R3[i];
            const float t2 = lsp + pr + R2[i];
            const float sp = omf(OMC_PS, k);
            const float t3 = lsp + sp + l1 + r2;
            const float t4 = lsp + sp + r1 + l2;
            const float m5 = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), t4);
            const float ms = fsafe(m5);
            const float s5 = exp2f(t0 - ms) + exp2f(t1 - ms) + exp2f(t2 - ms) + exp2f(t3 - ms) + exp2f(t4 - ms);
            lse_merge(dts[k], acc[k], m5, s5);
          }
        }
        __syncthreads();
      }
#pragma unroll
      for (int k = 0; k < CPT; ++k) dts[k] = log2f(acc[k]) + dts[k];
    }
    vst<CPT>(srow(SL_DTS), dts);

    // ---- 4. J^T coefficients at Pi* (wave_backward.py:264-416)
    ep = rr * 16 + 4;
    // p' = 2^(col + Pi* - rowmax).  The Pibar coefficient's denominator,
    // rowsum - pathsum(i) = the sum of p' over the non-ancestors of i (the
    // reference's ancestor chase, wave_backward.py:364-389), is the row's own
    // Pibar* in linear units, 2^(Pibar*_i - mt_i - rowmax): the forward's last
    // sweep wrote Pibar* from the same Pi*, so no scan is needed.  Pi* is in
    // R0 at preorder positions (the child gathers) since the row's staging,
    // unless the split term above restaged R0.
    float pp[CPT], pcoef[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = pos(k);
      pp[k] = i < S ? exp2_hw((WEIGHTED ? omf(OMC_COL, k) : 0.0f) + piv[k] - rms) : 0.0f;
      const float denom = i < S ? exp2_hw(pbv[k] - omf(OMC_MT, k) - rms) : 0.0f;
      pcoef[k] = denom > 0.0f ? rcp_hw(denom) : 0.0f;  // 1 / (rowsum - ps) for now
    }
    if (!leaf_row && !P.dts_in) {
      lds_store_own<CPT>(R0, piv);  // padding positions: -inf
      __syncthreads();
    }
    // diag = q0 + q1, pcoef = q2 / (rowsum - ps); child-edge weights into
    // position i from its parent (q3 if i is child1, else q4) scattered by the
    // parent's owner into R1 (Pibar* was read above), then read back.  The
    // barrier also ends the reads of R2 / R3, which become scan buffers.
    float diag[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = pos(k);
      diag[k] = 0.0f;
      if (i < S) {
        const int c1 = omi(OMT_C1, k), c2 = omi(OMT_C2, k);
        const Coef6 c = coef_at(coef_k(k), piv[k], pbv[k], dts[k], c1 >= 0 ? R0[c1] : KB_NEG_INF,
                                c2 >= 0 ? R0[c2] : KB_NEG_INF, leaf_row, i == lpos);
        diag[k] = c.q[0] + c.q[1];
        pcoef[k] = c.q[2] * pcoef[k];
        if (c1 >= 0) R1[c1] = c.q[3];
        if (c2 >= 0) R1[c2] = c.q[4];
      } else {
        pcoef[k] = 0.0f;
      }
    }
    __syncthreads();
    // parent position, subtree end - 1 and child-1 flag of each own position,
    // packed (OMT_PK)
    float edge[CPT];
    int pk[CPT];
    lds_load_own<CPT>(R1, edge);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      pk[k] = omi(OMT_PK, k);
      edge[k] = (pk[k] & 0xffff) != ZERO ? edge[k] : 0.0f;
    }
    // pk as values the optimiser cannot hoist out of the loops below (the LDS
    // addresses derived from it would otherwise stay live across them)
    auto pk_now = [&](int (&o)[CPT], int epoch) {
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        o[k] = pk[k];
        if constexpr (CPT > 4) asm("; %1" : "+v"(o[k]) : "s"(epoch));
      }
    };
    auto ppos_of = [](int x) { return x & 0xffff; };
    auto endm1_of = [](int x) { return (x >> 16) & 0x3fff; };
    auto wend_of = [](int x) { return (x >> (16 + SEGSH)) & (NW - 1); };  // ZERO -> wavefront 0

    // ---- 5. Neumann series v = sum_{n<=N} (J^T)^n rhs with the row on chip:
    // one barrier per term, buffers alternating by parity, and with EARLY the
    // same early stop as bwd_row_kernel (the series ends at the first term
    // with every entry at most rtol * max|rhs|; the wavefronts' votes travel
    // with their scan totals, in wt[NW + w])
    float v[CPT], term[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      v[k] = rhs[k];
      term[k] = rhs[k];
    }
    const float tau = P.rtol * row_amax;
    auto neumann_term = [&](float* Tb, float* Lb, float* wt, int n_term) -> bool {
      // the LDS addresses come from the packed tables in every term: held
      // across the loop they would take 3 x CPT registers
      int pkt[CPT];
      pk_now(pkt, n_term);
      float sc[CPT];
#pragma unroll
      for (int k = 0; k < CPT; ++k) sc[k] = term[k] * pcoef[k] + (k > 0 ? sc[k - 1] : 0.0f);
      const float tsum = sc[CPT - 1];
      const float ws = wave_scan_incl(tsum);
      if (lane == 63) wt[wv] = ws;
      if constexpr (EARLY) {
        bool small = true;
#pragma unroll
        for (int k = 0; k < CPT; ++k) small = small && fabsf(term[k]) <= tau;
        const bool all_small = __all(small);
        if (lane == 63) wt[NW + wv] = all_small ? 1.0f : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < CPT; ++k) sc[k] += ws - tsum;
      lds_store_own<CPT>(Lb, sc);
      lds_store_own<CPT>(Tb, term);
      __syncthreads();
      if constexpr (EARLY) {
        const float f = lane < NW ? wt[NW + lane] : 1.0f;
        if (__all(f != 0.0f)) return true;
      }
      float le[CPT], tpar[CPT];
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        le[k] = Lb[endm1_of(pkt[k])];
        tpar[k] = Tb[ppos_of(pkt[k])];
      }
      float A, woff, wexcl;
      scan_offsets(wt, A, woff, wexcl);
      const float p0 = wave_prev_lane(sc[CPT - 1]) + woff;
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const float pm1 = k == 0 ? p0 : sc[k - 1] + woff;
        const int we = wend_of(pkt[k]);
        const float nt = term[k] * diag[k] + pp[k] * (pm1 + (A - (le[k] + __shfl(wexcl, we, 64)))) + tpar[k] * edge[k];
        term[k] = nt;
        v[k] += nt;
      }
      return false;
    };
    // calls: terms whose buffers were written (the stopping term included)
    int calls = 0;
    {
      bool stopped = false;
      for (; calls + 2 <= P.n_terms; calls += 2) {
        if (neumann_term(R0, R2, wA, calls)) {
          calls += 1;
          stopped = true;
          break;
        }
        if (neumann_term(R1, R3, wB, calls + 1)) {
          calls += 2;
          stopped = true;
          break;
        }
      }
      if (!stopped && calls < P.n_terms) {
        stopped = neumann_term(R0, R2, wA, calls);
        calls += 1;
      }
      if (P.terms_out && tid == 0) P.terms_out[row] = (unsigned char)min(stopped ? calls - 1 : calls, 255);
    }

    ep = rr * 16 + 6;
    // ---- 6. self-loop column gradient and parameter buckets.  The buffers of
    // the next term's parity are free: Pi* goes back to its Tb buffer for the
    // recomputed coefficients' child gathers, the scan of u = v * pcoef to its
    // Lb buffer.
    {
      // the buffers the last term did not write (its readers may still be
      // reading its own)
      float* Pt = (calls & 1) ? R1 : R0;
      float* Pb = (calls & 1) ? R3 : R2;
      float* wt = (calls & 1) ? wB : wA;
      {
        float x[CPT];
        vld<CPT>(srow(SL_PI), x);
        lds_store_own<CPT>(Pt, x);
#pragma unroll
        for (int k = 0; k < CPT; ++k) x[k] = v[k] * pcoef[k];
        float sc[CPT];
        local_scan_publish<NT, CPT>(sc, x, Pb, wt);
        __syncthreads();
        float A, woff, wexcl;
        scan_offsets(wt, A, woff, wexcl);
        const float p0 = wave_prev_lane(sc[CPT - 1]) + woff;
        int pkt[CPT];
        pk_now(pkt, ep);
        // the column-gradient term p' (P(i-1) + A - P(end(i)-1)), in pcoef's
        // registers (pcoef is not needed after this)
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
          const float pm1 = k == 0 ? p0 : sc[k - 1] + woff;
          const float rest = A - (Pb[endm1_of(pkt[k])] + __shfl(wexcl, wend_of(pkt[k]), 64));
          pcoef[k] = pos(k) < S ? pp[k] * (pm1 + rest) : 0.0f;
        }
      }
      // a group's bucket loads are all issued before its stores (a load after a
      // store to the slot would wait for that store)
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        float4 bk[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) bk[j] = ld4(srow(j) + 4 * g);
        float pb4[4], dt4[4];
        vld<4>(srow(SL_PIBAR) + 4 * g, pb4);
        vld<4>(srow(SL_DTS) + 4 * g, dt4);
        const float4 pt4 = ld4(Pt + tid * CPT + 4 * g);  // own positions of Pi* (vector LDS read)
        float x[8][4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int k = 4 * g + kk;
          const int i = pos(k);
#pragma unroll
          for (int j = 0; j < 8; ++j) x[j][kk] = 0.0f;
          if (i < S) {
            const int c1 = omi(OMT_C1, k), c2 = omi(OMT_C2, k);
            const Coef6 c = coef_at(coef_k(k), f4(pt4, kk), pb4[kk], dt4[kk], c1 >= 0 ? Pt[c1] : KB_NEG_INF,
                                    c2 >= 0 ? Pt[c2] : KB_NEG_INF, leaf_row, i == lpos);
            const float aw0 = v[k] * c.q[0], aw1 = v[k] * c.q[1], aw2 = v[k] * c.q[2];
            const float aw3 = v[k] * c.q[3], aw4 = v[k] * c.q[4], aw5 = v[k] * c.q[5];
            x[0][kk] = aw0;
            x[1][kk] = aw3 + aw4 + aw5;
            x[2][kk] = aw0 + aw2;
            x[3][kk] = aw1;
            x[4][kk] = aw4;
            x[5][kk] = aw3;
            x[6][kk] = aw2;
            x[7][kk] = pcoef[k];
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) st4_add(srow(j) + 4 * g, bk[j], x[j]);
      }
    }

    // ---- 7. split adjoints into the child rows (staging, preorder layout)
    for (int si = sb; si < se; ++si) {
      const int lrow = P.split_l[si], rrow = P.split_r[si];
      const size_t l = (size_t)lrow * S, r = (size_t)rrow * S;
      const float lsp = P.split_lsp[si];
      const float rml = P.rowmax[lrow], rmr = P.rowmax[rrow];
      const float rmsl = fsafe(rml), rmsr = fsafe(rmr);
      ep = -4 * si - 1;
      __syncthreads();  // previous readers of R0..R3 are done
      stage(R0, P.pi + l);
      stage(R1, P.pi + r);
      stage(R2, P.pibar + l);
      stage(R3, P.pibar + r);
      __syncthreads();
      ep = -4 * si - 2;
      // pass 1 (own positions, four at a time): the five split-term shares
      // vd_j; vd3 / vd4 replace the own positions of the children's Pibar
      // rows (R2 / R3, read only at own positions) for the child positions'
      // parent reads; buckets 0, 1, 6 take vd0, vd3 + vd4, vd1 + vd2
      float av[CPT], bv[CPT], udl[CPT], udr[CPT], ppl[CPT], ppr[CPT];
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const float4 b0 = ld4(srow(0) + 4 * g), b1 = ld4(srow(1) + 4 * g), b6 = ld4(srow(6) + 4 * g);
        float pv4[4];
        vld<4>(srow(SL_PI) + 4 * g, pv4);
        // own positions of the four staged child rows (vector LDS reads)
        const float4 pl4 = ld4(R0 + tid * CPT + 4 * g), pr4 = ld4(R1 + tid * CPT + 4 * g);
        const float4 bl4 = ld4(R2 + tid * CPT + 4 * g), br4 = ld4(R3 + tid * CPT + 4 * g);
        float y0[4], y1[4], y2[4], d3[4], d4[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int k = 4 * g + kk;
          const int i = pos(k);
          float vd0 = 0.0f, vd1 = 0.0f, vd2 = 0.0f, vd3 = 0.0f, vd4 = 0.0f;
          udl[k] = udr[k] = ppl[k] = ppr[k] = 0.0f;
          if (i < S) {
            const int c1 = omi(OMT_C1, k), c2 = omi(OMT_C2, k);
            const float pl = f4(pl4, kk), pr = f4(pr4, kk), bl = f4(bl4, kk), br = f4(br4, kk);
            const float l1 = c1 >= 0 ? R0[c1] : KB_NEG_INF, r1 = c1 >= 0 ? R1[c1] : KB_NEG_INF;
            const float l2 = c2 >= 0 ? R0[c2] : KB_NEG_INF, r2 = c2 >= 0 ? R1[c2] : KB_NEG_INF;
            const float d = omf(OMC_PD, k), sp = omf(OMC_PS, k);
            const bool pv = pv4[kk] != KB_NEG_INF;
            const float base = pv ? lsp - pv4[kk] : 0.0f;
            vd0 = pv ? v[k] * exp2_hw(base + (d + pl + pr)) : 0.0f;
            vd1 = pv ? v[k] * exp2_hw(base + (pl + br)) : 0.0f;
            vd2 = pv ? v[k] * exp2_hw(base + (pr + bl)) : 0.0f;
            vd3 = pv ? v[k] * exp2_hw(base + (sp + l1 + r2)) : 0.0f;
            vd4 = pv ? v[k] * exp2_hw(base + (sp + r1 + l2)) : 0.0f;
            const float mts = omf(OMC_MT, k);
            const float inv_l = bl != KB_NEG_INF ? exp2_hw(rml + mts - bl) : 0.0f;
            const float inv_r = br != KB_NEG_INF ? exp2_hw(rmr + mts - br) : 0.0f;
            udl[k] = vd2 * inv_l;
            udr[k] = vd1 * inv_r;
            const float cw = WEIGHTED ? omf(OMC_COL, k) : 0.0f;
            ppl[k] = exp2_hw(cw + pl - rmsl);
            ppr[k] = exp2_hw(cw + pr - rmsr);
          }
          av[k] = vd0 + vd1;
          bv[k] = vd0 + vd2;
          y0[kk] = vd0;
          y1[kk] = vd3 + vd4;
          y2[kk] = vd1 + vd2;
          d3[kk] = vd3;
          d4[kk] = vd4;
        }
        *reinterpret_cast<float4*>(R2 + tid * CPT + 4 * g) = make_float4(d3[0], d3[1], d3[2], d3[3]);
        *reinterpret_cast<float4*>(R3 + tid * CPT + 4 * g) = make_float4(d4[0], d4[1], d4[2], d4[3]);
        st4_add(srow(0) + 4 * g, b0, y0);
        st4_add(srow(1) + 4 * g, b1, y1);
        st4_add(srow(6) + 4 * g, b6, y2);
      }
      __syncthreads();  // the staged children (R0, R1) fully read; vd3 / vd4 published
      float4 b7[NG];
#pragma unroll
      for (int g = 0; g < NG; ++g) b7[g] = ld4(srow(7) + 4 * g);
      float scl[CPT], scr[CPT];
      local_scan_publish<NT, CPT>(scl, udl, R0, wA);
      local_scan_publish<NT, CPT>(scr, udr, R1, wA + NW);
      __syncthreads();
      float Al, woffl, wexl, Ar, woffr, wexr;
      scan_offsets(wA, Al, woffl, wexl);
      scan_offsets(wA + NW, Ar, woffr, wexr);
      const float p0l = wave_prev_lane(scl[CPT - 1]) + woffl;
      const float p0r = wave_prev_lane(scr[CPT - 1]) + woffr;
      ep = -4 * si - 3;
      float* stl = P.staging + (size_t)(2 * si) * kb_stage_ld(S);
      float* str = P.staging + (size_t)(2 * si + 1) * kb_stage_ld(S);
      int pkt[CPT];
      pk_now(pkt, ep);
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        float y3[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int k = 4 * g + kk;
          const int i = pos(k);
          const int e1 = endm1_of(pkt[k]), we = wend_of(pkt[k]);
          const float pml = k == 0 ? p0l : scl[k - 1] + woffl;
          const float pmr = k == 0 ? p0r : scr[k - 1] + woffr;
          const float rsl = Al - (R0[e1] + __shfl(wexl, we, 64));
          const float rsr = Ar - (R1[e1] + __shfl(wexr, we, 64));
          y3[kk] = 0.0f;
          if (i < S) {
            const float tl = ppl[k] * (pml + rsl);
            const float tr = ppr[k] * (pmr + rsr);
            const int pa = ppos_of(pkt[k]);
            const bool first_child = (pkt[k] >> 30) & 1;
            const float sh3 = R2[pa], sh4 = R3[pa];  // padding slot holds 0
            const float shl = first_child ? sh3 : sh4;
            const float shr = first_child ? sh4 : sh3;
            stg(stl, i, av[k] + shl + tl);
            stg(str, i, bv[k] + shr + tr);
            y3[kk] = tl + tr;
          }
        }
        st4_add(srow(7) + 4 * g, b7[g], y3);
      }
      if (tid == 0) P.split_on[si] = 1;
    }
  }  // rows
}

#define KB_BWD_LARGE_CASE(NT_, CPT_)                                                                           \
  if (S <= NT_ * CPT_) {                                                                                       \
    const bool early = P.rtol > 0.0f;                                                                          \
    if (P.use_col && early)                                                                                    \
      hipLaunchKernelGGL((bwd_row_large_kernel<NT_, CPT_, true, true>), dim3(nb), dim3(NT_), 0, st, P, first, W, poff);   \
    else if (P.use_col)                                                                                        \
      hipLaunchKernelGGL((bwd_row_large_kernel<NT_, CPT_, true, false>), dim3(nb), dim3(NT_), 0, st, P, first, W, poff);  \
    else if (early)                                                                                            \
      hipLaunchKernelGGL((bwd_row_large_kernel<NT_, CPT_, false, true>), dim3(nb), dim3(NT_), 0, st, P, first, W, poff);  \
    else                                                                                                       \
      hipLaunchKernelGGL((bwd_row_large_kernel<NT_, CPT_, false, false>), dim3(nb), dim3(NT_), 0, st, P, first, W, poff); \
    return true;                                                                                               \
  }

bool launch_bwd_large(const BwdParams& P, int first, int W, int nb, int poff, hipStream_t st) {
  const int S = P.S;
  if (!kb_use_large(S, P.large)) return false;
  // the shape kb_large_nt / kb_large_ld give the owner-major tables
  if (kb_large_nt(S) == 512) {
    KB_BWD_LARGE_CASE(512, 4)
  }
  KB_BWD_LARGE_CASE(1024, 4)
  KB_BWD_LARGE_CASE(1024, 8)
  return false;
}

int bwd_large_blocks_per_cu(int S, int use_col) {
  int n = 0;
  auto occ = [&](auto kernel, int nt) { (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, nt, 0); };
  if (kb_large_nt(S) == 512)
    use_col ? occ(bwd_row_large_kernel<512, 4, true, false>, 512) : occ(bwd_row_large_kernel<512, 4, false, false>, 512);
  else if (S <= 4096)
    use_col ? occ(bwd_row_large_kernel<1024, 4, true, false>, 1024) : occ(bwd_row_large_kernel<1024, 4, false, false>, 1024);
  else
    use_col ? occ(bwd_row_large_kernel<1024, 8, true, false>, 1024) : occ(bwd_row_large_kernel<1024, 8, false, false>, 1024);
  return n > 0 ? n : 1;
}

}  // namespace kb
