// Fused backward: implicit-differentiation adjoint of the wave solve.
//
// Reference semantics (reference kbench/api/_implicit_grad.py:97-370 driving
// pristine wave_backward.py):
//   seed   rhs[root] = -2^(Pi*[root] - LSE2(Pi*[root]))           (_implicit_grad.py:151-158)
//   per wave, reverse order:
//     active[w] = max_s |rhs| >= thr  (> thr without pruning)      (wave_backward.py:138-201)
//     dts_r recomputed at Pi* with inactive parents at -inf        (_implicit_grad.py:206-227)
//     J^T coefficients at Pi* (diag, Pibar coefficient, p', child edges)
//                                                                  (wave_backward.py:203-416)
//     v = sum_{n=0..N} (J^T)^n rhs                                  (wave_backward.py:419-570, 1232-1269)
//     grad_col += sum p'(A - subtree(u)), u = v * pibar_coeff       (wave_backward.py:656-744)
//     buckets aw_k = v w_L e_k / sum e                              (wave_backward.py:747-966)
//     split adjoints into the child rows, incl. the Pibar VJP      (wave_backward.py:1529-1945, 2229-2327)
//
// One workgroup per clade row, rows scheduled by clade-DAG level in reverse.
// Threads own preorder positions (kb_rowops.hpp), where every subtree is a
// contiguous range: A - subtree(u)[i] = P[i-1] + (A - P[end(i)-1]) for the
// inclusive scan P of u over positions, one block scan per Neumann term.
//
// Latency: one workgroup per CU walks the level's rows persistently.  While
// a row is solved, the next row's data (its schedule-slot record, Pi* /
// Pibar* rows, child staging rows and split flags, row maxima and stored
// split term) is already in flight; seven per-position constant rows stay in
// LDS for the launch; the scans that need every wavefront publish
// wavefront-local values and let the readers add the wavefront offsets, so
// most phases take one barrier.
//
// Determinism: the reference scatters child adjoints and gradient sums with
// float atomics.  Here every split side writes a staging row (preorder
// layout); a child row gathers its staging rows in increasing split order,
// and every per-row gradient bucket is stored and reduced over rows in a fixed
// order, so results are bitwise reproducible.
#include <algorithm>
#include <type_traits>

#include "kb_device.hpp"
#include "kb_kernels.hpp"
#include "kb_rowops.hpp"

namespace kb {

// EARLY: the Neumann series may stop early (P.rtol > 0), a separate
// instantiation so that the loop without it keeps its own code and registers
template <int NT, int CPT, bool WEIGHTED, bool EARLY>
__global__ __launch_bounds__(NT) void bwd_row_kernel(BwdParams P, int first, int n_rows, int poff) {
  constexpr int MAXS = NT * CPT;
  constexpr int LD = MAXS + 64;  // [MAXS] is the padding slot, kept at 0
  constexpr int NW = NT / 64;
  __shared__ float L[4 * LD];
  __shared__ __align__(8) float wA[2 * NW], wB[2 * NW];
  __shared__ float wMk[NW];  // wavefront maxima of |adjoint| for the active mask
  float* R0 = L;
  float* R1 = L + LD;
  float* R2 = L + 2 * LD;
  float* R3 = L + 3 * LD;

  const PreDev& T = P.pre;
  const int S = P.S;
  const int tid = threadIdx.x;
  constexpr int ZERO = MAXS;

  // The 1024 x 2 shape (rows of 1025..2048 states on every level, shorter
  // rows on levels with about one row per workgroup) fetches rows when needed
  // instead of one row ahead (128 VGPRs at 16 waves).
  constexpr bool AHEAD = NT < 1024;
  // the first split's child rows are prefetched into registers during the
  // Neumann loop, except where 1024 threads (128 VGPRs) own four or more
  // positions each: there the registers spill to scratch memory
  constexpr bool PF = !(NT == 1024 && CPT >= 4);
  // The set-up's loads (the first row's record, the position tables, the
  // bucket slot, the constant rows) are all issued before any of them is
  // consumed, and the first row's fetch before the LDS stores that wait for
  // them: two memory round trips in all.
  const bool first_rec = AHEAD && !P.class_mode && (int)blockIdx.x < n_rows;
  const int rec0 = first_rec ? P.bslot[(size_t)KB_BREC * (first + blockIdx.x) + (tid & (KB_BREC - 1))] : 0;
  // The wide shape's set-up reads its per-position rows with one vector load
  // each (16-byte rows: the tables and constants start their allocations, the
  // slot rows are kb_slot_ld(S) floats apart); the narrow shape (128 VGPRs)
  // keeps one load per position, as the vector loads' registers spill there.
  constexpr bool VEC = NT < 1024;
  OwnTablesC<NT, CPT> O;
  O.template load<VEC>(T);
  if (tid < 64) {
    R0[MAXS + tid] = 0.0f;
    R1[MAXS + tid] = 0.0f;
    R2[MAXS + tid] = 0.0f;
    R3[MAXS + tid] = 0.0f;
  }
  bool okp[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) okp[k] = own_pos_c<NT, CPT>(k) < S;
  // static per position: parent position (ZERO at the root), child-1 flag,
  // subtree end - 1
  // and, for the root-path sums, the position at own postorder slot k (the
  // padding slot ZERO past the row) and tin(i) - i
  int ppos[CPT], endm1[CPT], pfl[CPT], qp[CPT], nex[CPT];
  if constexpr (VEC) {
    int tpa[CPT], tpf[CPT], tend[CPT];
    gld_own<CPT>(T.post, S, qp, ZERO);
    gld_own<CPT>(T.ppos, S, tpa, -1);
    gld_own<CPT>(T.pflag, S, tpf, 0);
    gld_own<CPT>(T.endpos, S, tend, ZERO + 1);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      nex[k] = okp[k] ? O.tin[k] - own_pos_c<NT, CPT>(k) : 0;
      ppos[k] = tpa[k] >= 0 ? tpa[k] : ZERO;
      pfl[k] = tpa[k] >= 0 ? tpf[k] : 0;
      endm1[k] = tend[k] - 1;
    }
  } else {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = own_pos_c<NT, CPT>(k);
      qp[k] = okp[k] ? T.post[i] : ZERO;
      nex[k] = okp[k] ? T.tin[i] - i : 0;
      const int pa = okp[k] ? T.ppos[i] : -1;
      const int pf = okp[k] ? T.pflag[i] : 0;  // loaded with ppos, not after it
      ppos[k] = pa >= 0 ? pa : ZERO;
      pfl[k] = pa >= 0 ? pf : 0;
      endm1[k] = okp[k] ? T.endpos[i] - 1 : ZERO;
    }
  }
  // gradient buckets of every row this workgroup processes (static round-robin
  // assignment, so the summation order is fixed), starting from this
  // workgroup's slot (preorder layout): slot b is carried by workgroup b of
  // every level in turn.  Its values are read here, with the other set-up
  // loads, and the launch ends with plain stores.
  // (in LDS for rows of up to 2048 states, own positions only: each thread
  // reads and writes just its own entries, so the accumulation needs no
  // barrier; in registers for longer rows, whose LDS rows leave no room)
  constexpr bool BK_LDS = MAXS <= 2048;
  __shared__ float Bk[BK_LDS ? 8 * MAXS : 1];
  float cacc[BK_LDS ? 1 : 8][CPT];
  // (slot rows are kb_slot_ld(S) floats apart, a multiple of four, so a
  // thread's positions are one vector access)
  const int SL = kb_slot_ld(S, 0);
  const int SG = kb_stage_ld(S);  // child staging rows likewise
  // (poff: the first slot of this launch's workgroups)
  float* const cr = P.contrib + (size_t)(poff + (int)blockIdx.x) * 8 * SL;
  float old[8][CPT];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (VEC) {
      gld_own<CPT>(cr + (size_t)j * SL, S, old[j], 0.0f);
    } else {
#pragma unroll
      for (int k = 0; k < CPT; ++k) old[j][k] = okp[k] ? cr[(size_t)j * SL + own_pos_c<NT, CPT>(k)] : 0.0f;
    }
  }
  // Per-position constants, one [S] row shared by every row: for rows of up
  // to 2048 states, seven of them stay in LDS for the whole launch (own
  // positions, so each thread reads back only what it wrote), and the per-row
  // coefficient passes read LDS instead of waiting on memory.  mt (and the
  // column weights) stay in memory: LDS has no room for an eighth row.
  constexpr bool CK_LDS = MAXS <= 2048;
  enum { K_DL, K_EBAR, K_E, K_SL1, K_SL2, K_PD, K_PS, K_N };
  __shared__ float Kc[CK_LDS ? K_N * MAXS : 1];
  const float* const kg[K_N] = {P.DL, P.Ebar, P.E, P.SL1, P.SL2, P.pD, P.pS};
  float kx[CK_LDS ? K_N : 1][CPT];
  if constexpr (CK_LDS) {
#pragma unroll
    for (int j = 0; j < K_N; ++j) {
      if constexpr (VEC) {
        gld_own<CPT>(kg[j], S, kx[j], 0.0f);
      } else {
#pragma unroll
        for (int k = 0; k < CPT; ++k) kx[j][k] = okp[k] ? kg[j][own_pos_c<NT, CPT>(k)] : 0.0f;
      }
    }
  }
  // constant j at own position k (0 at padding positions)
  auto kc_own = [&](int j, float (&x)[CPT]) {
    if constexpr (CK_LDS) {
      lds_load_own<CPT>(Kc + j * MAXS, x);
    } else {
#pragma unroll
      for (int k = 0; k < CPT; ++k) x[k] = okp[k] ? kg[j][own_pos_c<NT, CPT>(k)] : 0.0f;
    }
  };
  auto bucket = [&](int j, int k) -> float& {
    if constexpr (BK_LDS)
      return Bk[j * MAXS + own_pos_c<NT, CPT>(k)];
    else
      return cacc[j][k];
  };
  // buckets j[0..3] += x[0..3] at the own positions (vector LDS
  // read-modify-writes; the four reads are issued before the first write, so
  // their latencies overlap instead of queueing behind each write)
  auto bucket_add4 = [&](const int (&j)[4], const float (&x)[4][CPT]) {
    if constexpr (BK_LDS) {
      float cur[4][CPT];
#pragma unroll
      for (int b = 0; b < 4; ++b) lds_load_own<CPT>(Bk + j[b] * MAXS, cur[b]);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) cur[b][k] += x[b][k];
        lds_store_own<CPT>(Bk + j[b] * MAXS, cur[b]);
      }
    } else {
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int k = 0; k < CPT; ++k) cacc[j[b]][k] += x[b][k];
    }
  };

  // What a row needs from memory is fetched one row ahead, while the previous
  // row is solved: Pi* / Pibar* (column s = tid + j*NT to registers, then to
  // its preorder position spre[j] in LDS), and below the class level the
  // row's record (BrecField, lanes 0..KB_BREC-1), the split_on flags and
  // staging rows of its first two child sides (whose active sum, in side
  // order, is the adjoint; further sides, rare, are gathered when the row
  // starts), the row maxima of the row and of its first split's children, and
  // its stored split term.  Flags and maxima are vector loads (lanes 0..2
  // hold the different entries), so the LDS waits in between do not wait on
  // them.  The narrow shape fetches all of it when the row starts.
  auto row_of = [&](int r2) { return P.class_mode ? P.cls_rows[P.cls_ptr[r2]] : P.sched_rows[first + r2]; };
  int spre[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int s = tid + j * NT;
    spre[j] = s < S ? T.pre[s] : -1;
  }
  float nPi[CPT], nPb[CPT];
  auto fetch_rows = [&](int row2) {
    const size_t b2 = (size_t)row2 * S;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int s = tid + j * NT;
      nPi[j] = spre[j] >= 0 ? P.pi[b2 + s] : 0.0f;
      nPb[j] = spre[j] >= 0 ? P.pibar[b2 + s] : 0.0f;
    }
  };
  auto load_rec = [&](int r2) -> int { return P.bslot[(size_t)KB_BREC * (first + r2) + (tid & (KB_BREC - 1))]; };
  // (read fields at uniform points only: a lane read inside divergent code may
  // see a register that was restored for the active lanes alone)
  auto field = [](int rec, int f) { return __builtin_amdgcn_readlane(rec, f); };
  float nst0[CPT], nst1[CPT], nds[CPT], nrm = 0.0f;
  int nfl = 0;
  auto fetch_row_data = [&](int rec) {
    const int s0 = field(rec, BR_S0), s1r = field(rec, BR_S1);
    const int s1 = s1r < 0 ? -1 : (s1r & ((1 << 30) - 1));
    const int sl = (tid & 1) ? s1 : s0;
    nfl = sl >= 0 ? (int)P.split_on[sl >> 1] : 0;
    const int frow = field(rec, BR_ROW), fl0 = field(rec, BR_L0), fr0 = field(rec, BR_R0);
    const int leaf = field(rec, BR_LEAF), rep = field(rec, BR_REP);
    const int q = tid & 3;
    const int rmr = q == 0 ? frow : q == 1 ? fl0 : fr0;
    nrm = rmr >= 0 ? P.rowmax[rmr] : 0.0f;
    const bool dts = !leaf && P.dts_in;
    const size_t db = (size_t)rep * S;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = own_pos_c<NT, CPT>(k);
      if constexpr (!VEC) {
        nst0[k] = (s0 >= 0 && okp[k]) ? P.staging[(size_t)s0 * SG + i] : 0.0f;
        nst1[k] = (s1 >= 0 && okp[k]) ? P.staging[(size_t)s1 * SG + i] : 0.0f;
      }
      nds[k] = (dts && okp[k]) ? P.dts_in[db + i] : KB_NEG_INF;
    }
    if constexpr (VEC) {
      // one unchecked vector load per row (the allocation's tail covers the
      // positions past S, whose values are dropped where the rows are added;
      // a side that does not exist reads row 0 and its flag is 0): a
      // bounds-checked load would join into a register copy that waits here
      // for every load just issued
      static_assert(MAXS <= KB_STAGE_TAIL && CPT % 2 == 0, "staging tail, vector width");
      auto ld_row = [&](const float* row, float (&v)[CPT]) {
        if constexpr (CPT % 4 == 0) {
#pragma unroll
          for (int g = 0; g < CPT / 4; ++g) {
            const float4 x = reinterpret_cast<const float4*>(row)[tid * (CPT / 4) + g];
            v[4 * g] = x.x, v[4 * g + 1] = x.y, v[4 * g + 2] = x.z, v[4 * g + 3] = x.w;
          }
        } else {
#pragma unroll
          for (int g = 0; g < CPT / 2; ++g) {
            const float2 x = reinterpret_cast<const float2*>(row)[tid * (CPT / 2) + g];
            v[2 * g] = x.x, v[2 * g + 1] = x.y;
          }
        }
      };
      ld_row(P.staging + (size_t)max(s0, 0) * SG, nst0);
      ld_row(P.staging + (size_t)max(s1, 0) * SG, nst1);
    }
  };
  // The 1024 x 2 shape reads its rows' records from LDS: RCH of them at a
  // time, one int per thread (KB_BREC fields of RCH rows), the first chunk
  // with the set-up loads; a row then waits for one memory round trip (its
  // data) instead of two (its record, then its data).
  constexpr int RCH = 1024 / KB_BREC;
  __shared__ int Rec[AHEAD ? 1 : RCH * KB_BREC];
  auto load_chunk = [&](int rr2) {
    if constexpr (!AHEAD) {
      static_assert(NT == RCH * KB_BREC, "one record field per thread");
      const int r2 = rr2 + (tid / KB_BREC) * (int)gridDim.x;
      Rec[tid] = r2 < n_rows ? P.bslot[(size_t)KB_BREC * (first + r2) + (tid & (KB_BREC - 1))] : 0;
    }
  };
  if (!AHEAD && !P.class_mode) load_chunk(blockIdx.x);
  int ci = 0;  // (1024 x 2) this row's entry in the chunk
  int crec = 0, nrec = 0;  // records of the next two rows (AHEAD, below the class level)
  if (AHEAD && (int)blockIdx.x < n_rows) {
    if (P.class_mode) {
      fetch_rows(row_of(blockIdx.x));
    } else {
      crec = rec0;
      fetch_rows(field(crec, BR_ROW));
      fetch_row_data(crec);
      nrec = load_rec(min((int)(blockIdx.x + gridDim.x), n_rows - 1));
    }
  }
  // the next row's fetches (AHEAD, below the class level).  Unconditional,
  // with clamped slots (past the last row they fetch a row again, unused): a
  // conditional load would join into a register copy that waits for every
  // load just issued.
  auto advance = [&](int rr2) {
    crec = nrec;
    nrec = load_rec(min(rr2 + 2 * (int)gridDim.x, n_rows - 1));
    fetch_rows(field(crec, BR_ROW));
    fetch_row_data(crec);
  };
  // the set-up's LDS stores, after every load above is in flight
  if constexpr (CK_LDS) {
#pragma unroll
    for (int j = 0; j < K_N; ++j) lds_store_own<CPT>(Kc + j * MAXS, kx[j]);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      if constexpr (BK_LDS)
        Bk[j * MAXS + own_pos_c<NT, CPT>(k)] = old[j][k];
      else
        cacc[j][k] = old[j][k];
    }

  for (int rr = blockIdx.x; rr < n_rows; rr += gridDim.x) {
  __syncthreads();  // LDS of the previous row is no longer read
  const int cm = P.class_mode;
  int rec = 0;
  if constexpr (AHEAD) {
    rec = cm ? 0 : crec;
  } else if (!cm) {
    if (ci == 0 && rr != (int)blockIdx.x) {  // uniform: the next chunk
      load_chunk(rr);
      __syncthreads();
    }
    rec = Rec[ci * KB_BREC + (tid & (KB_BREC - 1))];
    ci = (ci + 1) & (RCH - 1);
  }
  // every field read here, at a uniform point
  const int f_row = field(rec, BR_ROW), f_leaf = field(rec, BR_LEAF), f_sb = field(rec, BR_SB);
  const int f_se = field(rec, BR_SE), f_fam = field(rec, BR_FAM), f_s1 = field(rec, BR_S1);
  const int f_lpos = field(rec, BR_LPOS), f_l0 = field(rec, BR_L0), f_r0 = field(rec, BR_R0);
  const float f_lsp0 = __int_as_float(field(rec, BR_LSP0));
  const int row = cm ? row_of(rr) : f_row;
  const int leaf_row = cm ? P.row_kind[row] : f_leaf;
  const int sb = cm ? P.split_ptr[row] : f_sb, se = cm ? P.split_ptr[row + 1] : f_se;
  if (!AHEAD) {
    fetch_rows(row);
    if (!cm) fetch_row_data(rec);
  }

  // ---- 1. Pi* of this row; adjoint = root seed or fixed-order gather of the
  // staging rows.  In class mode (identical rows without splits) each member's
  // adjoint gets its own active-mask decision and the active members' adjoints
  // are summed: everything below is linear in the adjoint.
  // The adjoint gathers are issued first, then Pi* and Pibar* go through LDS to
  // preorder positions under one barrier, so the three loads overlap.
  float rhs[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) rhs[k] = 0.0f;
  bool any_active = false;
  const int fam = cm ? -1 : f_fam;
  if (P.class_mode) {
    // the summed adjoint of the class's active members (bwd_gather0 / bwd_classsum0)
    any_active = P.cls_active[rr] != 0;
    const float* src = P.rhsc + (size_t)rr * S;
#pragma unroll
    for (int k = 0; k < CPT; ++k)
      if (okp[k]) rhs[k] = src[own_pos_c<NT, CPT>(k)];
  } else {
    if (__builtin_amdgcn_readlane(nfl, 0)) {
#pragma unroll
      for (int k = 0; k < CPT; ++k) rhs[k] += okp[k] ? nst0[k] : 0.0f;
    }
    if (__builtin_amdgcn_readlane(nfl, 1)) {
#pragma unroll
      for (int k = 0; k < CPT; ++k) rhs[k] += okp[k] ? nst1[k] : 0.0f;
    }
    if (f_s1 >= 0 && (f_s1 >> 30) != 0) {  // more than two child sides
      const int gb = P.child_ptr[row] + 2, ge = P.child_ptr[row + 1];
      for (int i = gb; i < ge; ++i) {
        const int side = P.child_in[i];
        if (!P.split_on[side >> 1]) continue;
        const float* st = P.staging + (size_t)side * SG;
#pragma unroll
        for (int k = 0; k < CPT; ++k)
          if (okp[k]) rhs[k] += st[own_pos_c<NT, CPT>(k)];
      }
    }
  }
  // rows below the roots: their adjoint is known here, so the wavefront maxima
  // for the active mask are published under the staging barrier below
  const bool mask_early = !P.class_mode && fam < 0;
  // (class rows publish them too when the Neumann series may stop early: its
  // threshold is relative to the row's largest adjoint entry)
  if (mask_early || (EARLY && P.class_mode)) {
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) am = fmaxf(am, fabsf(rhs[k]));
    const float wm = wave_reduce_max(am);
    if ((tid & 63) == 0) wMk[tid >> 6] = wm;
  }
  float piv[CPT], pbv[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j)
    if (spre[j] >= 0) {
      R0[spre[j]] = nPi[j];
      R1[spre[j]] = nPb[j];
    }
  if (AHEAD && cm && rr + (int)gridDim.x < n_rows) fetch_rows(row_of(rr + gridDim.x));
  __syncthreads();
  lds_load_own<CPT>(R0, piv);
  lds_load_own<CPT>(R1, pbv);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    if (!okp[k]) piv[k] = pbv[k] = KB_NEG_INF;
  }
  float row_amax = 0.0f;  // max |adjoint| of the row
  if (EARLY && P.class_mode) {
#pragma unroll
    for (int w = 0; w < NW; ++w) row_amax = fmaxf(row_amax, wMk[w]);
  }
  if (!P.class_mode) {
    if (fam >= 0) {
      // logsumexp2 (logspace.py:11-16) and _safe_exp2_ratio (_implicit_grad.py:21-25)
      float lm = KB_NEG_INF;
#pragma unroll
      for (int k = 0; k < CPT; ++k) lm = fmaxf(lm, piv[k]);
      const float rmax = block_max1<NT>(lm, wA);
      const float rms = fsafe(rmax);
      float ls = 0.0f;
#pragma unroll
      for (int k = 0; k < CPT; ++k) ls += okp[k] ? exp2f(piv[k] - rms) : 0.0f;
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
  // row data of this row that is read after the next row's fetches
  const float rms = fsafe(cm ? P.rowmax[row] : lane_value(nrm, 0));
  const float rml0 = cm ? 0.0f : lane_value(nrm, 1), rmr0 = cm ? 0.0f : lane_value(nrm, 2);
  if (!any_active) {
    for (int i = sb + tid; i < se; i += NT) P.split_on[i] = 0;
    if (AHEAD && !cm) advance(rr);
    continue;
  }
  // The root rows' reductions above used the scratch that the path sums
  // reuse, and the split term below (without stored split terms) restages
  // R0..R3: those wait for every wavefront here.  Otherwise each thread has
  // read only its own positions of R0 / R1 since the staging barrier.
  if (fam >= 0 || (!leaf_row && !P.dts_in)) __syncthreads();

  // ---- 3. split term at Pi* (split rows), children staged through LDS
  float dts[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) dts[k] = KB_NEG_INF;
  if (!leaf_row && P.dts_in) {
    if (cm) {
      const float* src = P.dts_in + (size_t)P.rep_of[row] * S;
#pragma unroll
      for (int k = 0; k < CPT; ++k)
        if (okp[k]) dts[k] = src[own_pos_c<NT, CPT>(k)];
    } else {
#pragma unroll
      for (int k = 0; k < CPT; ++k) dts[k] = nds[k];
    }
  } else if (!leaf_row) {
    float m[CPT], acc[CPT], kd[CPT], ks[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      m[k] = KB_NEG_INF;
      acc[k] = 0.0f;
    }
    kc_own(K_PD, kd);
    kc_own(K_PS, ks);
    for (int si = sb; si < se; ++si) {
      const size_t l = (size_t)P.split_l[si] * S, r = (size_t)P.split_r[si] * S;
      const float lsp = P.split_lsp[si];
#pragma unroll
      for (int j = 0; j < CPT; ++j)
        if (spre[j] >= 0) {
          const int s = tid + j * NT;
          R0[spre[j]] = P.pi[l + s];
          R1[spre[j]] = P.pi[r + s];
          R2[spre[j]] = P.pibar[l + s];
          R3[spre[j]] = P.pibar[r + s];
        }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int i = own_pos_c<NT, CPT>(k);
        if (okp[k]) {
          const bool h1 = O.c1p[k] != ZERO, h2 = O.c2p[k] != ZERO;
          const float pl = R0[i], pr = R1[i];
          const float d = kd[k], sp = ks[k];
          const float l1 = h1 ? R0[O.c1p[k]] : KB_NEG_INF, r1 = h1 ? R1[O.c1p[k]] : KB_NEG_INF;
          const float l2 = h2 ? R0[O.c2p[k]] : KB_NEG_INF, r2 = h2 ? R1[O.c2p[k]] : KB_NEG_INF;
          const float t0 = lsp + d + pl + pr;
          const float t1 = lsp + pl + R3[i];
          const float t2 = lsp + pr + R2[i];
          const float t3 = lsp + sp + l1 + r2;
          const float t4 = lsp + sp + r1 + l2;
          const float m5 = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), t4);
          const float ms = fsafe(m5);
          const float s5 = exp2f(t0 - ms) + exp2f(t1 - ms) + exp2f(t2 - ms) + exp2f(t3 - ms) + exp2f(t4 - ms);
          lse_merge(m[k], acc[k], m5, s5);
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k) dts[k] = log2f(acc[k]) + m[k];
  }

  // ---- 4. J^T coefficients at Pi* (precompute kernel, wave_backward.py:264-416)
  // p' = 2^(col + Pi* - rowmax).  The Pibar coefficient's denominator,
  // rowsum - pathsum(i) = the sum of p' over the non-ancestors of i (the
  // reference's ancestor chase, wave_backward.py:364-389), is the row's own
  // Pibar* in linear units: Pibar*_i = log2(sum_{j not anc(i)} 2^(col_j +
  // Pi*_j)) + mt_i, written by the forward's last sweep from the same Pi*, so
  // the sum is 2^(Pibar*_i - mt_i - rowmax) and needs no scan.  Pi* is in R0
  // at preorder positions (the child gathers) since the row's staging, unless
  // the split-term recompute restaged R0.
  float pp[CPT], pmt[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = own_pos_c<NT, CPT>(k);
    pp[k] = okp[k] ? exp2_hw((WEIGHTED ? P.col[i] : 0.0f) + piv[k] - rms) : 0.0f;
    pmt[k] = okp[k] ? P.mt[i] : 0.0f;
  }
  const int wv = tid >> 6, lane = tid & 63;
  if (!leaf_row && !P.dts_in) {
    lds_store_own<CPT>(R0, piv);  // padding positions: -inf
    __syncthreads();
  }
  const int lpos = cm ? (leaf_row ? T.pre[P.leaf_state[row]] : -1) : f_lpos;
  float q[6][CPT], pcoef[CPT];
  float kDL[CPT], kEb[CPT], kE[CPT], kS1[CPT], kS2[CPT], kLf[CPT];
  kc_own(K_DL, kDL);
  kc_own(K_EBAR, kEb);
  kc_own(K_E, kE);
  kc_own(K_SL1, kS1);
  kc_own(K_SL2, kS2);
  kc_own(K_PS, kLf);  // the leaf term's log pS
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = own_pos_c<NT, CPT>(k);
#pragma unroll
    for (int j = 0; j < 6; ++j) q[j][k] = 0.0f;
    pcoef[k] = 0.0f;
    if (okp[k]) {
      const float denom = exp2_hw(pbv[k] - pmt[k] - rms);
      const float inv_denom = denom > 0.0f ? rcp_hw(denom) : 0.0f;
      const bool h1 = O.c1p[k] != ZERO, h2 = O.c2p[k] != ZERO;
      const float t0 = kDL[k] + piv[k];
      const float t1 = piv[k] + kEb[k];
      const float t2 = pbv[k] + kE[k];
      const float t3 = kS1[k] + (h1 ? R0[O.c1p[k]] : KB_NEG_INF);
      const float t4 = kS2[k] + (h2 ? R0[O.c2p[k]] : KB_NEG_INF);
      const float t5 = i == lpos ? kLf[k] : KB_NEG_INF;
      const float m = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), fmaxf(t4, t5));
      const float msf = fsafe(m);
      float e[6] = {exp2_hw(t0 - msf), exp2_hw(t1 - msf), exp2_hw(t2 - msf), exp2_hw(t3 - msf),
                    exp2_hw(t4 - msf), exp2_hw(t5 - msf)};
      const float sum = e[0] + e[1] + e[2] + e[3] + e[4] + e[5];
      // q_j = w_L e_j / sum with the split mixing weight
      // w_L = 2^dl / (2^dl + 2^dts), 2^dl = sum 2^m:  q_j = e_j / (sum + 2^(dts - m))
      const float den = sum + (leaf_row ? 0.0f : exp2_hw(dts[k] - msf));
      const float inv = sum > 0.0f ? rcp_hw(den) : 0.0f;
#pragma unroll
      for (int j = 0; j < 6; ++j) q[j][k] = e[j] * inv;
      pcoef[k] = q[2][k] * inv_denom;
    }
  }
  // child-edge weights into position i from its parent: q3 if i is child1,
  // else q4.  The parent's owner scatters them into R1 (free since Pibar* was
  // read; every position has one parent, the root none), one barrier, and
  // each thread reads its own positions.
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    if (O.c1p[k] != ZERO) R1[O.c1p[k]] = q[3][k];
    if (O.c2p[k] != ZERO) R1[O.c2p[k]] = q[4][k];
  }
  __syncthreads();
  float edge[CPT], diag[CPT];
  lds_load_own<CPT>(R1, edge);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    edge[k] = ppos[k] != ZERO ? edge[k] : 0.0f;
    diag[k] = q[0][k] + q[1][k];
  }

  // The first split's four child rows (Pi, Pibar of both children) are loaded
  // into registers here, so their latency overlaps the Neumann loop.
  float pf[4][CPT];
  if (PF && se > sb) {
    const size_t l = (size_t)(cm ? P.split_l[sb] : f_l0) * S;
    const size_t r = (size_t)(cm ? P.split_r[sb] : f_r0) * S;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int s = tid + j * NT;
      const bool ok = s < S;
      pf[0][j] = ok ? P.pi[l + s] : 0.0f;
      pf[1][j] = ok ? P.pi[r + s] : 0.0f;
      pf[2][j] = ok ? P.pibar[l + s] : 0.0f;
      pf[3][j] = ok ? P.pibar[r + s] : 0.0f;
    }
  }

  // ---- 5. Neumann series v = sum_{n<=N} (J^T)^n rhs with the row on chip
  float v[CPT], term[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    v[k] = rhs[k];
    term[k] = rhs[k];
  }
  // One barrier per term.  The scan of u = term * pcoef is published
  // wavefront-local (a per-thread running sum plus one wavefront scan of the
  // thread totals); after the barrier each wavefront offset comes from the
  // published totals (lanes 0..NW-1, one more wavefront scan), so
  // P[j] = L[j] + off(wavefront of j).  P[i - 1] comes from the thread itself,
  // the previous lane, or the offset; P[end(i) - 1] and the parent's term are
  // read back.  Buffers alternate by parity, so the next term's writes never
  // race this term's reads.
  //
  // Stopping early (P.rtol > 0): the series ends at the first term n whose
  // every entry is at most rtol * max|rhs| (the row's threshold tau); that
  // term is already in v and J^T of it is not formed (a term n = 0 can pass
  // only if rhs is zero).  Every adjoint entry has the sign of the root seeds
  // (rhs <= 0, J^T and the split adjoints have nonnegative coefficients), so
  // |v| >= |rhs| entrywise and the dropped remainder is below rtol of the
  // row's largest adjoint entry times the tail's geometric factor.  Each
  // wavefront publishes its vote with its scan total (wt[2w], wt[2w + 1]),
  // under the term's barrier, and every thread reads all votes with the
  // totals, so all take the same decision.  The loop without the early stop
  // is a separate kernel instantiation, with the totals at wt[w].
  int wend[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) wend[k] = endm1[k] < ZERO ? endm1[k] / (64 * CPT) : 0;
  const float tau = P.rtol * row_amax;
  // term n uses the buffers of its parity; the loop runs the terms in pairs
  // so that every LDS address is a register plus a constant.  With the early
  // stop (EARLY) a term returns true when the series stops at it.
  auto neumann_term = [&](float* Tb, float* Lb, float* wt) -> bool {
    float sc[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) sc[k] = term[k] * pcoef[k] + (k > 0 ? sc[k - 1] : 0.0f);
    const float tsum = sc[CPT - 1];
    const float ws = wave_scan_incl(tsum);
    if constexpr (EARLY) {
      bool small = true;
#pragma unroll
      for (int k = 0; k < CPT; ++k) small = small && fabsf(term[k]) <= tau;
      const float vote = __all(small) ? 1.0f : 0.0f;
      if (lane == 63) reinterpret_cast<float2*>(wt)[wv] = make_float2(ws, vote);
    } else {
      if (lane == 63) wt[wv] = ws;
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k) sc[k] += ws - tsum;  // wavefront-local inclusive scan
    lds_store_own<CPT>(Lb, sc);
    lds_store_own<CPT>(Tb, term);
    __syncthreads();
    float le[CPT], tpar[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      le[k] = Lb[endm1[k]];
      tpar[k] = Tb[ppos[k]];
    }
    float wtot;
    if constexpr (EARLY) {
      const float2 tv = lane < NW ? reinterpret_cast<const float2*>(wt)[lane] : make_float2(0.0f, 1.0f);
      if (__all(tv.y != 0.0f)) return true;
      wtot = tv.x;
    } else {
      wtot = lane < NW ? wt[lane] : 0.0f;
    }
    const float wincl = wave_scan_first<NW>(wtot);
    const float wexcl = wincl - wtot;                 // lane x < NW: offset of wavefront x
    const float A = lane_value(wincl, NW - 1);
    const float woff = lane_value(wexcl, wv);         // this wavefront's offset
    const float p0 = wave_prev_lane(sc[CPT - 1]) + woff;  // P[i - 1] of slot 0
    float oe[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) oe[k] = __shfl(wexcl, wend[k], 64);
    __builtin_amdgcn_sched_barrier(0);  // all permutes in flight before the first use
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const float pm1 = k == 0 ? p0 : sc[k - 1] + woff;
      const float nt = term[k] * diag[k] + pp[k] * (pm1 + (A - (le[k] + oe[k]))) + tpar[k] * edge[k];
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
      if (neumann_term(R0, R2, wA)) {
        calls += 1;
        stopped = true;
        break;
      }
      if (neumann_term(R1, R3, wB)) {
        calls += 2;
        stopped = true;
        break;
      }
    }
    if (!stopped && calls < P.n_terms) {
      stopped = neumann_term(R0, R2, wA);
      calls += 1;
    }
    if (P.terms_out && tid == 0) P.terms_out[row] = (unsigned char)min(stopped ? calls - 1 : calls, 255);
  }

  if (AHEAD && !cm) advance(rr);
  // mt at the own positions for the split adjoints (its load overlaps the
  // self-loop gradient and the child staging)
  float kmt[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) kmt[k] = okp[k] ? P.mt[own_pos_c<NT, CPT>(k)] : 0.0f;

  // ---- 6. self-loop column gradient and parameter buckets
  {
    // the buffers the last term did not write (its readers may still be
    // reading its own)
    float* Pb = (calls & 1) ? R3 : R2;
    float* wt = (calls & 1) ? wB : wA;
    float u[CPT], sc[CPT], pm1[CPT], rest[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) u[k] = v[k] * pcoef[k];
    local_scan_publish<NT, CPT>(sc, u, Pb, wt);
    __syncthreads();
    subtree_terms<NT, CPT>(sc, Pb, wt, endm1, wend, pm1, rest);
    float x[2][4][CPT];  // buckets 0..3, 4..7
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const float aw0 = v[k] * q[0][k], aw1 = v[k] * q[1][k], aw2 = v[k] * q[2][k];
      const float aw3 = v[k] * q[3][k], aw4 = v[k] * q[4][k], aw5 = v[k] * q[5][k];
      x[0][0][k] = aw0;
      x[0][1][k] = aw3 + aw4 + aw5;
      x[0][2][k] = aw0 + aw2;
      x[0][3][k] = aw1;
      x[1][0][k] = aw4;
      x[1][1][k] = aw3;
      x[1][2][k] = aw2;
      x[1][3][k] = okp[k] ? pp[k] * (pm1[k] + rest[k]) : 0.0f;
    }
    bucket_add4({0, 1, 2, 3}, x[0]);
    bucket_add4({4, 5, 6, 7}, x[1]);
  }

  // ---- 7. split adjoints into the child rows (staging, preorder layout)
  for (int si = sb; si < se; ++si) {
    const bool s0 = si == sb && !cm;  // the first split's data came with the row
    const int lrow = s0 ? f_l0 : P.split_l[si], rrow = s0 ? f_r0 : P.split_r[si];
    const size_t l = (size_t)lrow * S, r = (size_t)rrow * S;
    const float lsp = s0 ? f_lsp0 : P.split_lsp[si];
    const float rml = s0 ? rml0 : P.rowmax[lrow], rmr = s0 ? rmr0 : P.rowmax[rrow];
    const float rmsl = fsafe(rml), rmsr = fsafe(rmr);
    __syncthreads();  // previous readers of R0..R3 are done
    if (PF && si == sb) {
#pragma unroll
      for (int j = 0; j < CPT; ++j)
        if (spre[j] >= 0) {
          R0[spre[j]] = pf[0][j];
          R1[spre[j]] = pf[1][j];
          R2[spre[j]] = pf[2][j];
          R3[spre[j]] = pf[3][j];
        }
    } else {
#pragma unroll
      for (int j = 0; j < CPT; ++j)
        if (spre[j] >= 0) {
          const int s = tid + j * NT;
          R0[spre[j]] = P.pi[l + s];
          R1[spre[j]] = P.pi[r + s];
          R2[spre[j]] = P.pibar[l + s];
          R3[spre[j]] = P.pibar[r + s];
        }
    }
    __syncthreads();
    float vd0[CPT], vd1[CPT], vd2[CPT], vd3[CPT], vd4[CPT], udl[CPT], udr[CPT], ppl[CPT], ppr[CPT];
    float cPl[CPT], cPr[CPT], cBl[CPT], cBr[CPT], kd[CPT], ks[CPT];
    kc_own(K_PD, kd);
    kc_own(K_PS, ks);
    lds_load_own<CPT>(R0, cPl);
    lds_load_own<CPT>(R1, cPr);
    lds_load_own<CPT>(R2, cBl);
    lds_load_own<CPT>(R3, cBr);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = own_pos_c<NT, CPT>(k);
      vd0[k] = vd1[k] = vd2[k] = vd3[k] = vd4[k] = udl[k] = udr[k] = ppl[k] = ppr[k] = 0.0f;
      if (okp[k]) {
        const bool h1 = O.c1p[k] != ZERO, h2 = O.c2p[k] != ZERO;
        const float pl = cPl[k], pr = cPr[k], bl = cBl[k], br = cBr[k];
        const float l1 = h1 ? R0[O.c1p[k]] : KB_NEG_INF, r1 = h1 ? R1[O.c1p[k]] : KB_NEG_INF;
        const float l2 = h2 ? R0[O.c2p[k]] : KB_NEG_INF, r2 = h2 ? R1[O.c2p[k]] : KB_NEG_INF;
        const float d = kd[k], sp = ks[k];
        const bool pv = piv[k] != KB_NEG_INF;
        const float base = pv ? lsp - piv[k] : 0.0f;
        vd0[k] = pv ? v[k] * exp2_hw(base + (d + pl + pr)) : 0.0f;
        vd1[k] = pv ? v[k] * exp2_hw(base + (pl + br)) : 0.0f;
        vd2[k] = pv ? v[k] * exp2_hw(base + (pr + bl)) : 0.0f;
        vd3[k] = pv ? v[k] * exp2_hw(base + (sp + l1 + r2)) : 0.0f;
        vd4[k] = pv ? v[k] * exp2_hw(base + (sp + r1 + l2)) : 0.0f;
        const float mts = kmt[k];
        const float inv_l = bl != KB_NEG_INF ? exp2_hw(rml + mts - bl) : 0.0f;
        const float inv_r = br != KB_NEG_INF ? exp2_hw(rmr + mts - br) : 0.0f;
        udl[k] = vd2[k] * inv_l;
        udr[k] = vd1[k] * inv_r;
        const float cw = WEIGHTED ? P.col[i] : 0.0f;
        ppl[k] = exp2_hw(cw + pl - rmsl);
        ppr[k] = exp2_hw(cw + pr - rmsr);
      }
    }
    __syncthreads();  // staged children fully read
    lds_store_own<CPT>(R0, vd3);
    lds_store_own<CPT>(R1, vd4);
    float scl[CPT], scr[CPT], pml[CPT], rsl[CPT], pmr[CPT], rsr[CPT];
    local_scan_publish<NT, CPT>(scl, udl, R2, wA);
    local_scan_publish<NT, CPT>(scr, udr, R3, wA + NW);
    __syncthreads();
    subtree_terms<NT, CPT>(scl, R2, wA, endm1, wend, pml, rsl);
    subtree_terms<NT, CPT>(scr, R3, wA + NW, endm1, wend, pmr, rsr);
    float* stl = P.staging + (size_t)(2 * si) * SG;
    float* str = P.staging + (size_t)(2 * si + 1) * SG;
    float y[4][CPT], ysl[CPT], ysr[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      // (padding positions: every operand below is 0 there, and so are the
      // values; their parent slot ppos holds 0)
      const float tl = ppl[k] * (pml[k] + rsl[k]);
      const float tr = ppr[k] * (pmr[k] + rsr[k]);
      const int pa = ppos[k];
      const bool first = pfl[k] != 0;
      const float sh3 = R0[pa], sh4 = R1[pa];  // padding slot holds 0
      const float shl = first ? sh3 : sh4;
      const float shr = first ? sh4 : sh3;
      ysl[k] = okp[k] ? vd0[k] + vd1[k] + shl + tl : 0.0f;
      ysr[k] = okp[k] ? vd0[k] + vd2[k] + shr + tr : 0.0f;
      y[0][k] = vd0[k];
      y[1][k] = vd3[k] + vd4[k];
      y[2][k] = vd1[k] + vd2[k];
      y[3][k] = okp[k] ? tl + tr : 0.0f;
    }
    if constexpr (VEC) {
      gst_own<CPT>(stl, S, ysl);
      gst_own<CPT>(str, S, ysr);
    } else {
#pragma unroll
      for (int k = 0; k < CPT; ++k)
        if (okp[k]) {
          stl[own_pos_c<NT, CPT>(k)] = ysl[k];
          str[own_pos_c<NT, CPT>(k)] = ysr[k];
        }
    }
    bucket_add4({0, 1, 6, 7}, y);
    if (tid == 0) P.split_on[si] = 1;
  }

  }  // rows

  // this workgroup's slot holds the buckets carried through this level
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (VEC) {
      float x[CPT];
#pragma unroll
      for (int k = 0; k < CPT; ++k) x[k] = bucket(j, k);
      gst_own<CPT>(cr + (size_t)j * SL, S, x);
    } else {
#pragma unroll
      for (int k = 0; k < CPT; ++k)
        if (okp[k]) cr[(size_t)j * SL + own_pos_c<NT, CPT>(k)] = bucket(j, k);
    }
  }
}

#define KB_BWD_CASE(NT_, CPT_)                                                                        \
  if (S <= NT_ * CPT_) {                                                                              \
    const bool early = P.rtol > 0.0f;                                                                 \
    if (P.use_col && early)                                                                           \
      hipLaunchKernelGGL((bwd_row_kernel<NT_, CPT_, true, true>), dim3(nb), dim3(NT_), 0, st, P, first, W, poff);   \
    else if (P.use_col)                                                                               \
      hipLaunchKernelGGL((bwd_row_kernel<NT_, CPT_, true, false>), dim3(nb), dim3(NT_), 0, st, P, first, W, poff);  \
    else if (early)                                                                                   \
      hipLaunchKernelGGL((bwd_row_kernel<NT_, CPT_, false, true>), dim3(nb), dim3(NT_), 0, st, P, first, W, poff);  \
    else                                                                                              \
      hipLaunchKernelGGL((bwd_row_kernel<NT_, CPT_, false, false>), dim3(nb), dim3(NT_), 0, st, P, first, W, poff); \
    return;                                                                                           \
  }

// Level-0 rows, in two passes:
//  gather0   one workgroup per member: adjoint row (root seed or fixed-order
//            gather of its live staging rows; the side lists are static,
//            m_side_ptr / m_side in member order) in preorder positions, and
//            its active mask (in member order, m_mask, and per row, mask);
//  classsum0 per (class, 256-position block): the sum in member order of the
//            class's active members' rows.
constexpr int G0_E = 8;  // positions per thread per pass of gather0

__global__ __launch_bounds__(256) void bwd_gather0_kernel(BwdParams P) {
  __shared__ float red[4];
  const PreDev& T = P.pre;
  const int S = P.S;
  const int mi = blockIdx.x;
  const int row = P.cls_rows[mi];
  const int sb = P.m_side_ptr[mi], se = P.m_side_ptr[mi + 1];
  float* out = P.rhs0 + (size_t)mi * S;
  float am = 0.0f;
  if (P.m_root[mi] >= 0) {
    // root seed: -2^(Pi - logsumexp2(Pi)) (logspace.py:11-16, _implicit_grad.py:21-25)
    const float* pr = P.pi + (size_t)row * S;
    float lm = KB_NEG_INF;
    for (int j = threadIdx.x; j < S; j += 256) lm = fmaxf(lm, pr[j]);
    const float rmax = block_max<256>(lm, red);
    const float rms = fsafe(rmax);
    float ls = 0.0f;
    for (int j = threadIdx.x; j < S; j += 256) ls += exp2f(pr[j] - rms);
    const float tot = block_sum<256>(ls, red);
    const float lses = fsafe((tot > 0.0f ? log2f(tot) : KB_NEG_INF) + rmax);
    for (int i = threadIdx.x; i < S; i += 256) {
      const float x = pr[T.col[i]];
      const float r = x == KB_NEG_INF ? 0.0f : -exp2f(x - lses);
      out[i] = r;
      am = fmaxf(am, fabsf(r));
    }
  } else {
    for (int base = 0; base < S; base += 256 * G0_E) {
      float r[G0_E];
#pragma unroll
      for (int e = 0; e < G0_E; ++e) r[e] = 0.0f;
      for (int j = sb; j < se; ++j) {
        const int side = P.m_side[j];
        if (!P.split_on[side >> 1]) continue;  // uniform across the workgroup
        const float* st = P.staging + (size_t)side * kb_stage_ld(S);
#pragma unroll
        for (int e = 0; e < G0_E; ++e) {
          const int i = base + e * 256 + threadIdx.x;
          if (i < S) r[e] += st[i];
        }
      }
#pragma unroll
      for (int e = 0; e < G0_E; ++e) {
        const int i = base + e * 256 + threadIdx.x;
        if (i < S) {
          out[i] = r[e];
          am = fmaxf(am, fabsf(r[e]));
        }
      }
    }
  }
  const float amax = block_max<256>(am, red);
  if (threadIdx.x == 0) {
    const unsigned char on = (P.use_pruning ? (amax >= P.thr) : (amax > P.thr)) ? 1 : 0;
    P.mask[row] = on;
    P.m_mask[mi] = on;
  }
}

__global__ __launch_bounds__(256) void bwd_classsum0_kernel(BwdParams P) {
  __shared__ unsigned char on[256];
  const int c = blockIdx.x;
  const int S = P.S;
  const int i = blockIdx.y * 256 + threadIdx.x;
  const int mb = P.cls_ptr[c], me = P.cls_ptr[c + 1];
  float acc = 0.0f;
  int any = 0;
  for (int m0 = mb; m0 < me; m0 += 256) {
    const int n = min(256, me - m0);
    __syncthreads();
    if (threadIdx.x < n) on[threadIdx.x] = P.m_mask[m0 + threadIdx.x];
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      if (!on[j]) continue;
      any = 1;
      if (i < S) acc += P.rhs0[(size_t)(m0 + j) * S + i];
    }
  }
  if (i < S) P.rhsc[(size_t)c * S + i] = acc;
  if (blockIdx.y == 0 && threadIdx.x == 0) P.cls_active[c] = any ? 1 : 0;
}

// Level-0 adjoints for trees of up to 256 * G0_E nodes, one workgroup per
// chunk of a class's members (at most KB_CHUNK0): each member's adjoint row
// stays in registers (position e*256 + tid), gets its active mask, and the
// active members are summed in member order into the chunk's partial row
// (kept in the rhs0 buffer).  bwd_chunksum0_kernel then adds a class's chunk
// rows in chunk order.  Same per-member arithmetic as bwd_gather0_kernel,
// without the [members, S] round trip through HBM.
__global__ __launch_bounds__(256) void bwd_chunk0_kernel(BwdParams P) {
  __shared__ float red[4];
  __shared__ float wmax[KB_CHUNK0][4];
  const PreDev& T = P.pre;
  const int S = P.S;
  const int tid = threadIdx.x;
  const int k = blockIdx.x;
  const int mb = P.ck_ptr[k], me = P.ck_ptr[k + 1];
  // Every member's adjoint row stays in registers: all members' staging loads
  // are issued before the first reduction, and one barrier gives every
  // member's mask.
  float r[KB_CHUNK0][G0_E];
  bool has_root = false;
#pragma unroll
  for (int m = 0; m < KB_CHUNK0; ++m) {
#pragma unroll
    for (int e = 0; e < G0_E; ++e) r[m][e] = 0.0f;
    const int mi = mb + m;
    if (mi >= me) continue;
    if (P.m_root[mi] >= 0) {
      has_root = true;
      continue;
    }
    for (int j = P.m_side_ptr[mi]; j < P.m_side_ptr[mi + 1]; ++j) {
      const int side = P.m_side[j];
      const bool on = P.split_on[side >> 1] != 0;  // uniform across the workgroup
      const float* st = P.staging + (size_t)side * kb_stage_ld(S);
#pragma unroll
      for (int e = 0; e < G0_E; ++e) {
        const int i = e * 256 + tid;
        const float x = i < S ? st[i] : 0.0f;
        r[m][e] = on ? r[m][e] + x : r[m][e];
      }
    }
  }
  if (has_root) {
    // root seeds -2^(Pi - logsumexp2(Pi)) (logspace.py:11-16, _implicit_grad.py:21-25)
#pragma unroll
    for (int m = 0; m < KB_CHUNK0; ++m) {
      const int mi = mb + m;
      if (mi >= me || P.m_root[mi] < 0) continue;
      const float* pr = P.pi + (size_t)P.cls_rows[mi] * S;
      float lm = KB_NEG_INF;
      for (int j = tid; j < S; j += 256) lm = fmaxf(lm, pr[j]);
      const float rmax = block_max<256>(lm, red);
      const float rms = fsafe(rmax);
      float ls = 0.0f;
      for (int j = tid; j < S; j += 256) ls += exp2f(pr[j] - rms);
      const float tot = block_sum<256>(ls, red);
      const float lses = fsafe((tot > 0.0f ? log2f(tot) : KB_NEG_INF) + rmax);
#pragma unroll
      for (int e = 0; e < G0_E; ++e) {
        const int i = e * 256 + tid;
        if (i < S) {
          const float x = pr[T.col[i]];
          r[m][e] = x == KB_NEG_INF ? 0.0f : -exp2f(x - lses);
        }
      }
    }
  }
  // the members' active masks (the reference's rule), one barrier
#pragma unroll
  for (int m = 0; m < KB_CHUNK0; ++m) {
    float am = 0.0f;
#pragma unroll
    for (int e = 0; e < G0_E; ++e)
      if (e * 256 + tid < S) am = fmaxf(am, fabsf(r[m][e]));
    const float wm = wave_reduce_max(am);
    if ((tid & 63) == 0) wmax[m][tid >> 6] = wm;
  }
  __syncthreads();
  float acc[G0_E];
#pragma unroll
  for (int e = 0; e < G0_E; ++e) acc[e] = 0.0f;
  int any = 0;
#pragma unroll
  for (int m = 0; m < KB_CHUNK0; ++m) {
    const int mi = mb + m;
    if (mi >= me) continue;
    const float amax = fmaxf(fmaxf(wmax[m][0], wmax[m][1]), fmaxf(wmax[m][2], wmax[m][3]));
    const bool on = P.use_pruning ? (amax >= P.thr) : (amax > P.thr);
    if (tid == 0) {
      P.mask[P.cls_rows[mi]] = on ? 1 : 0;
      P.m_mask[mi] = on ? 1 : 0;
    }
    if (on) {
      any = 1;
#pragma unroll
      for (int e = 0; e < G0_E; ++e) acc[e] += r[m][e];
    }
  }
  float* out = P.rhs0 + (size_t)k * S;
#pragma unroll
  for (int e = 0; e < G0_E; ++e) {
    const int i = e * 256 + tid;
    if (i < S) out[i] = acc[e];
  }
  if (tid == 0) P.ck_any[k] = any ? 1 : 0;
}

__global__ __launch_bounds__(256) void bwd_chunksum0_kernel(BwdParams P) {
  const int c = blockIdx.x;
  const int S = P.S;
  const int i = blockIdx.y * 256 + threadIdx.x;
  const int kb = P.cls_ck_ptr[c], ke = P.cls_ck_ptr[c + 1];
  float acc = 0.0f;
  int any = 0;
  for (int k = kb; k < ke; ++k) {
    any |= P.ck_any[k];
    if (i < S) acc += P.rhs0[(size_t)k * S + i];
  }
  if (i < S) P.rhsc[(size_t)c * S + i] = acc;
  if (blockIdx.y == 0 && threadIdx.x == 0) P.cls_active[c] = any ? 1 : 0;
}

void launch_bwd_level0_prep(const BwdParams& P, int n_members, int n_cls, hipStream_t st) {
  if (n_members <= 0) return;
  const int nblk = (P.S + 255) / 256;
  if (P.S <= 256 * G0_E && P.n_chunks0 > 0) {
    hipLaunchKernelGGL(bwd_chunk0_kernel, dim3(P.n_chunks0), dim3(256), 0, st, P);
    hipLaunchKernelGGL(bwd_chunksum0_kernel, dim3(n_cls, nblk), dim3(256), 0, st, P);
    return;
  }
  hipLaunchKernelGGL(bwd_gather0_kernel, dim3(n_members), dim3(256), 0, st, P);
  hipLaunchKernelGGL(bwd_classsum0_kernel, dim3(n_cls, nblk), dim3(256), 0, st, P);
}

void launch_bwd_wave(const BwdParams& P, int first, int W, int nb, int poff, hipStream_t st) {
  if (W <= 0 || nb <= 0) return;
  if (launch_bwd_large(P, first, W, nb, poff, st)) return;
  const int S = P.S;
  if (P.variant == 2) {
    KB_BWD_CASE(1024, 2)
  }
  KB_BWD_CASE(64, 2)
  KB_BWD_CASE(128, 2)
  KB_BWD_CASE(256, 2)
  KB_BWD_CASE(256, 4)
  KB_BWD_CASE(512, 4)
  KB_BWD_CASE(1024, 4)
  KB_BWD_CASE(1024, 8)
}

#define KB_BWD_OCC(NT_, CPT_)                                                                          \
  if (S <= NT_ * CPT_) {                                                                               \
    int n = 0;                                                                                         \
    if (use_col)                                                                                       \
      (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, bwd_row_kernel<NT_, CPT_, true, false>, NT_, 0);  \
    else                                                                                               \
      (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, bwd_row_kernel<NT_, CPT_, false, false>, NT_, 0); \
    return n > 0 ? n : 1;                                                                              \
  }

int bwd_blocks_per_cu(int S, int use_col, int variant, int large) {
  if (kb_use_large(S, large)) return bwd_large_blocks_per_cu(S, use_col);
  if (variant == 2) {
    KB_BWD_OCC(1024, 2)
  }
  KB_BWD_OCC(64, 2)
  KB_BWD_OCC(128, 2)
  KB_BWD_OCC(256, 2)
  KB_BWD_OCC(256, 4)
  KB_BWD_OCC(512, 4)
  KB_BWD_OCC(1024, 4)
  KB_BWD_OCC(1024, 8)
  return 1;
}

// ---- backward constants from the saved tensors, in the glue's float32 order
// (_implicit_grad.py:136-143: DL = 1 + pD + E, SL1 = pS + E_s2, SL2 = pS + E_s1),
// written at preorder positions for the row kernel.
__global__ __launch_bounds__(256) void bwd_consts_kernel(BwdConstArgs A) {
  for (size_t z = (size_t)blockIdx.x * 256 + threadIdx.x; z < A.n_zero; z += (size_t)gridDim.x * 256) A.zero[z] = 0.0f;
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= A.S) return;
  const int i = A.pre[s];
  const float pS = A.log_pS[A.statewise ? s : 0];
  const float pD = A.log_pD[A.statewise ? s : 0];
  const float dl = (1.0f + pD) + A.E[s], sl1 = pS + A.E_s2[s], sl2 = pS + A.E_s1[s];
  A.DL[i] = dl;
  A.SL1[i] = sl1;
  A.SL2[i] = sl2;
  A.pS_state[i] = pS;
  A.pD_state[i] = pD;
  A.Ebar_pre[i] = A.Ebar[s];
  A.E_pre[i] = A.E[s];
  A.mt_pre[i] = A.mt[s];
  A.col_pre[i] = A.col[s];
  if (A.om) {
    const int ld = kb_large_ld(A.S), nt = kb_large_nt(A.S), cpt = ld / nt;
    float* o = A.om + (i % cpt) * nt + i / cpt;
    o[OMC_DL * ld] = dl;
    o[OMC_EBAR * ld] = A.Ebar[s];
    o[OMC_E * ld] = A.E[s];
    o[OMC_SL1 * ld] = sl1;
    o[OMC_SL2 * ld] = sl2;
    o[OMC_PD * ld] = pD;
    o[OMC_PS * ld] = pS;
    o[OMC_MT * ld] = A.mt[s];
    o[OMC_COL * ld] = A.col[s];
  }
}

void launch_bwd_consts(const BwdConstArgs& A, hipStream_t st) {
  const size_t zb = std::min<size_t>(4096, (A.n_zero + 255) / 256);
  hipLaunchKernelGGL(bwd_consts_kernel, dim3((unsigned)std::max<size_t>((A.S + 255) / 256, zb)), dim3(256), 0, st, A);
}

// ---- column sums of the per-row buckets over active rows, fixed order.
// Stage 1: chunk c of rows -> partial[c][8*S] at preorder positions;
// stage 2: sum of chunks, written in column order: out[j*S + s].
constexpr int RED_CHUNK = 16;

__global__ void bwd_reduce_stage1(const float* contrib, int C, int S, size_t slot_stride, int ld, double* partial) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;  // index in [0, 8S)
  const int chunk = blockIdx.y;
  if (j >= 8 * S) return;
  const int a = j / S;
  const size_t off = (size_t)a * ld + (j - a * S);
  const int r0 = chunk * RED_CHUNK, r1 = min(C, r0 + RED_CHUNK);
  double acc = 0.0;
  for (int r = r0; r < r1; ++r) acc += (double)contrib[(size_t)r * slot_stride + off];
  partial[(size_t)chunk * 8 * S + j] = acc;
}

// Entry j = a * S + s of out (accumulator a, column s) sums the chunk
// partials of its preorder position pre[s] in chunk order: the reduction and
// the return from preorder to column order in one pass.
__global__ void bwd_reduce_stage2(const double* partial, int n_chunks, int S, const int* pre, double* out) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= 8 * S) return;
  const int a = j / S, s = j - a * S;
  const size_t src = (size_t)a * S + pre[s];
  double acc = 0.0;
  for (int c = 0; c < n_chunks; ++c) acc += partial[(size_t)c * 8 * S + src];
  out[j] = acc;
}

void launch_bwd_reduce(const float* contrib, int C, int S, size_t slot_stride, int ld, double* partial, const int* pre,
                       double* out, hipStream_t st) {
  const int n_chunks = (C + RED_CHUNK - 1) / RED_CHUNK;
  dim3 g1((8 * S + 255) / 256, n_chunks);
  hipLaunchKernelGGL(bwd_reduce_stage1, g1, dim3(256), 0, st, contrib, C, S, slot_stride, ld, partial);
  hipLaunchKernelGGL(bwd_reduce_stage2, dim3((8 * S + 255) / 256), dim3(256), 0, st, partial, n_chunks, S, pre, out);
}

int reduce_chunks(int C) { return (C + RED_CHUNK - 1) / RED_CHUNK; }

}  // namespace kb
