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
// Determinism: the reference scatters child adjoints and gradient sums with
// float atomics.  Here every split side writes a staging row; a child row
// gathers its staging rows in increasing split order when its own wave runs,
// and every per-row gradient bucket is stored and reduced over rows in a
// fixed order, so results are bitwise reproducible.
#include "kb_device.hpp"
#include "kb_kernels.hpp"

namespace kb {

// Two subtree sums at once (same level schedule, half the barriers).
template <int NT>
__device__ __forceinline__ void subtree_sum2_lds(const TreeDev& tr, float* u, float* w) {
  for (int lv = 0; lv < tr.n_blevels; ++lv) {
    const int b = tr.blevel_ptr[lv], e = tr.blevel_ptr[lv + 1];
    for (int i = b + threadIdx.x; i < e; i += NT) {
      const int p = tr.blevel_node[i];
      const int x = tr.c1[p], y = tr.c2[p];
      u[p] += (x >= 0 ? u[x] : 0.0f) + (y >= 0 ? u[y] : 0.0f);
      w[p] += (x >= 0 ? w[x] : 0.0f) + (y >= 0 ? w[y] : 0.0f);
    }
    __syncthreads();
  }
}

template <int NT>
__device__ __forceinline__ void block_sum2(float& a, float& b, float* red) {
  constexpr int NW = NT / 64;
  a = wave_sum(a);
  b = wave_sum(b);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) {
    red[w] = a;
    red[NW + w] = b;
  }
  __syncthreads();
  float ra = red[0], rb = red[NW];
#pragma unroll
  for (int i = 1; i < NW; ++i) {
    ra += red[i];
    rb += red[NW + i];
  }
  __syncthreads();
  a = ra;
  b = rb;
}

template <int NT, int CPT>
__global__ __launch_bounds__(NT) void bwd_wave_kernel(BwdParams P, int first) {
  constexpr int MAXS = NT * CPT;
  __shared__ float B0[MAXS];
  __shared__ float B1[MAXS];
  __shared__ float B2[MAXS];
  __shared__ float B3[MAXS];
  __shared__ float red[2 * (NT / 64)];

  const int S = P.S;
  const int tid = threadIdx.x;
  const int row = P.sched_rows[first + blockIdx.x];
  const int leaf_wave = P.row_kind[row];
  const int item = P.item[row];
  const size_t cb = (size_t)item * P.const_stride;
  const size_t rb = (size_t)row * S;
  const int sb = P.split_ptr[row], se = P.split_ptr[row + 1];

  // ---- 1. adjoint of this row: root seed or fixed-order gather of staging rows
  float piv[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = tid + k * NT;
    piv[k] = s < S ? P.pi[rb + s] : KB_NEG_INF;
  }
  float rhs[CPT];
  const int fam = P.root_index[row];
  if (fam >= 0) {
    // logsumexp2 (logspace.py:11-16) and _safe_exp2_ratio (_implicit_grad.py:21-25)
    float lm = KB_NEG_INF;
#pragma unroll
    for (int k = 0; k < CPT; ++k) lm = fmaxf(lm, piv[k]);
    const float rmax = block_max<NT>(lm, red);
    const float rms = fsafe(rmax);
    float ls = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k)
      if (tid + k * NT < S) ls += exp2f(piv[k] - rms);
    const float tot = block_sum<NT>(ls, red);
    const float lse = (tot > 0.0f ? log2f(tot) : KB_NEG_INF) + rmax;
#pragma unroll
    for (int k = 0; k < CPT; ++k)
      rhs[k] = (piv[k] == KB_NEG_INF) ? 0.0f : -exp2f(piv[k] - (lse == KB_NEG_INF ? 0.0f : lse));
  } else {
#pragma unroll
    for (int k = 0; k < CPT; ++k) rhs[k] = 0.0f;
    const int gb = P.child_ptr[row], ge = P.child_ptr[row + 1];
    for (int i = gb; i < ge; ++i) {
      const int side = P.child_in[i];
      if (!P.split_on[side >> 1]) continue;
      const float* st = P.staging + (size_t)side * S;
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int s = tid + k * NT;
        if (s < S) rhs[k] += st[s];
      }
    }
  }

  // ---- 2. active mask (bit-exact rule of the reference)
  float am = 0.0f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) am = fmaxf(am, fabsf(rhs[k]));
  const float amax = block_max<NT>(am, red);
  const bool active = P.use_pruning ? (amax >= P.thr) : (amax > P.thr);
  if (tid == 0) P.mask[row] = active ? 1 : 0;
  if (!active) {
    for (int i = sb + tid; i < se; i += NT) P.split_on[i] = 0;
    return;
  }

  // ---- 3. split term at Pi* (split rows)
  float dts[CPT];
  if (!leaf_wave) {
    float m[CPT], acc[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      m[k] = KB_NEG_INF;
      acc[k] = 0.0f;
    }
    for (int i = sb; i < se; ++i) {
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
    for (int k = 0; k < CPT; ++k) dts[k] = log2f(acc[k]) + m[k];
  }

  // ---- 4. J^T coefficients at Pi* (precompute kernel)
  const float rms = fsafe(P.rowmax[row]);
  float pp[CPT];
  float ls = 0.0f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = tid + k * NT;
    pp[k] = 0.0f;
    if (s < S) {
      pp[k] = exp2f((P.use_col ? P.col[s] + piv[k] : piv[k]) - rms);
      B0[s] = pp[k];
      B2[s] = piv[k];
      ls += pp[k];
    }
  }
  const float rowsum = block_sum<NT>(ls, red);
  const float* ps = path_sum_lds<NT, CPT>(P.tr, B0, B1);
  const int leaf = leaf_wave ? P.leaf_state[row] : -1;
  float q[6][CPT], inv_denom[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = tid + k * NT;
#pragma unroll
    for (int j = 0; j < 6; ++j) q[j][k] = 0.0f;
    inv_denom[k] = 0.0f;
    if (s < S) {
      const float denom = rowsum - ps[s];
      inv_denom[k] = denom > 0.0f ? 1.0f / denom : 0.0f;
      const int a1 = P.tr.c1[s], a2 = P.tr.c2[s];
      const float t0 = P.DL[cb + s] + piv[k];
      const float t1 = piv[k] + P.Ebar[cb + s];
      const float t2 = P.pibar[rb + s] + P.E[cb + s];
      const float t3 = P.SL1[cb + s] + (a1 >= 0 ? B2[a1] : KB_NEG_INF);
      const float t4 = P.SL2[cb + s] + (a2 >= 0 ? B2[a2] : KB_NEG_INF);
      const float t5 = (leaf_wave && s == leaf) ? P.leaf_logp[cb + s] : KB_NEG_INF;
      float m = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), fmaxf(t4, t5));
      const float msf = fsafe(m);
      float e[6] = {exp2f(t0 - msf), exp2f(t1 - msf), exp2f(t2 - msf), exp2f(t3 - msf), exp2f(t4 - msf),
                    exp2f(t5 - msf)};
      const float sum = e[0] + e[1] + e[2] + e[3] + e[4] + e[5];
      const float inv_sum = sum > 0.0f ? 1.0f / sum : 0.0f;
      float wL = 1.0f;
      if (!leaf_wave) {
        const float dl = log2f(sum) + m;
        const float pm = fmaxf(dl, dts[k]);
        const float pms = fsafe(pm);
        const float pnew = log2f(exp2f(dl - pms) + exp2f(dts[k] - pms)) + pm;
        wL = dl == KB_NEG_INF ? 0.0f : exp2f(dl - pnew);
      }
#pragma unroll
      for (int j = 0; j < 6; ++j) q[j][k] = wL * e[j] * inv_sum;
    }
  }
  __syncthreads();  // B2 / path-sum buffers are reused below
  // child-edge weights: into column s from its parent p, q3[p] if s == c1[p] else q4[p]
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = tid + k * NT;
    if (s < S) {
      B0[s] = q[3][k];
      B1[s] = q[4][k];
    }
  }
  __syncthreads();
  float edge[CPT];
  int par[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = tid + k * NT;
    edge[k] = 0.0f;
    par[k] = -1;
    if (s < S) {
      const int p = P.tr.parent[s];
      par[k] = p;
      if (p >= 0) edge[k] = (P.tr.c1[p] == s) ? B0[p] : B1[p];
    }
  }
  __syncthreads();

  // ---- 5. Neumann series v = sum_{n<=N} (J^T)^n rhs, row on chip
  float v[CPT], term[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    v[k] = rhs[k];
    term[k] = rhs[k];
  }
  for (int n = 0; n < P.n_terms; ++n) {
    float lu = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      if (s < S) {
        const float u = term[k] * (q[2][k] * inv_denom[k]);
        B0[s] = term[k];
        B1[s] = u;
        lu += u;
      }
    }
    const float A = block_sum<NT>(lu, red);
    subtree_sum_lds<NT>(P.tr, B1);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      if (s < S) {
        float nt = term[k] * (q[0][k] + q[1][k]) + pp[k] * (A - B1[s]);
        if (par[k] >= 0) nt += B0[par[k]] * edge[k];
        term[k] = nt;
        v[k] += nt;
      }
    }
    __syncthreads();
  }

  // ---- 6. column gradient of the self loop and the parameter buckets
  float c[8][CPT];
  {
    float lu = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      if (s < S) {
        const float u = v[k] * (q[2][k] * inv_denom[k]);
        B1[s] = u;
        lu += u;
      }
    }
    const float A = block_sum<NT>(lu, red);
    subtree_sum_lds<NT>(P.tr, B1);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      const float aw0 = v[k] * q[0][k], aw1 = v[k] * q[1][k], aw2 = v[k] * q[2][k];
      const float aw3 = v[k] * q[3][k], aw4 = v[k] * q[4][k], aw5 = v[k] * q[5][k];
      c[0][k] = aw0;
      c[1][k] = aw3 + aw4 + aw5;
      c[2][k] = aw0 + aw2;
      c[3][k] = aw1;
      c[4][k] = aw4;
      c[5][k] = aw3;
      c[6][k] = aw2;
      c[7][k] = s < S ? pp[k] * (A - B1[s]) : 0.0f;
    }
    __syncthreads();
  }

  // ---- 7. split adjoints into the child rows (staging) incl. the Pibar VJP
  for (int i = sb; i < se; ++i) {
    const int lrow = P.split_l[i], rrow = P.split_r[i];
    const size_t l = (size_t)lrow * S, r = (size_t)rrow * S;
    const float lsp = P.split_lsp[i];
    const float* Pl = P.pi + l;
    const float* Pr = P.pi + r;
    const float* Bl = P.pibar + l;
    const float* Br = P.pibar + r;
    const float rml = P.rowmax[lrow], rmr = P.rowmax[rrow];
    float vd0[CPT], vd1[CPT], vd2[CPT];
    float al = 0.0f, ar = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      vd0[k] = vd1[k] = vd2[k] = 0.0f;
      if (s < S) {
        const int a1 = P.tr.c1[s], a2 = P.tr.c2[s];
        const float pl = Pl[s], pr = Pr[s], bl = Bl[s], br = Br[s];
        const float d = P.pD.at(item, s), sp = P.pS.at(item, s);
        const float l1 = a1 >= 0 ? Pl[a1] : KB_NEG_INF, r1 = a1 >= 0 ? Pr[a1] : KB_NEG_INF;
        const float l2 = a2 >= 0 ? Pl[a2] : KB_NEG_INF, r2 = a2 >= 0 ? Pr[a2] : KB_NEG_INF;
        const float pp_ = piv[k];
        const bool pv = pp_ != KB_NEG_INF;
        const float base = pv ? lsp - pp_ : 0.0f;
        const float w0 = pv ? exp2f(base + (d + pl + pr)) : 0.0f;
        const float w1 = pv ? exp2f(base + (pl + br)) : 0.0f;
        const float w2 = pv ? exp2f(base + (pr + bl)) : 0.0f;
        const float w3 = pv ? exp2f(base + (sp + l1 + r2)) : 0.0f;
        const float w4 = pv ? exp2f(base + (sp + r1 + l2)) : 0.0f;
        vd0[k] = v[k] * w0;
        vd1[k] = v[k] * w1;
        vd2[k] = v[k] * w2;
        const float vd3 = v[k] * w3, vd4 = v[k] * w4;
        B2[s] = vd3;
        B3[s] = vd4;
        const float mts = P.mt[cb + s];
        const float inv_l = bl != KB_NEG_INF ? exp2f(rml + mts - bl) : 0.0f;
        const float inv_r = br != KB_NEG_INF ? exp2f(rmr + mts - br) : 0.0f;
        const float udl = vd2[k] * inv_l, udr = vd1[k] * inv_r;
        B0[s] = udl;
        B1[s] = udr;
        al += udl;
        ar += udr;
        c[0][k] += vd0[k];
        c[1][k] += vd3 + vd4;
        c[6][k] += vd1[k] + vd2[k];
      }
    }
    block_sum2<NT>(al, ar, red);
    subtree_sum2_lds<NT>(P.tr, B0, B1);
    float* stl = P.staging + (size_t)(2 * i) * S;
    float* str = P.staging + (size_t)(2 * i + 1) * S;
    const float rmsl = fsafe(rml), rmsr = fsafe(rmr);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      if (s < S) {
        const float cw = P.use_col ? P.col[s] : 0.0f;
        const float ppl = exp2f(cw + Pl[s] - rmsl);
        const float ppr = exp2f(cw + Pr[s] - rmsr);
        const float tl = ppl * (al - B0[s]);
        const float tr = ppr * (ar - B1[s]);
        float shl = 0.0f, shr = 0.0f;
        const int p = par[k];
        if (p >= 0) {
          if (P.tr.c1[p] == s) {
            shl = B2[p];
            shr = B3[p];
          } else {
            shl = B3[p];
            shr = B2[p];
          }
        }
        stl[s] = vd0[k] + vd1[k] + shl + tl;
        str[s] = vd0[k] + vd2[k] + shr + tr;
        c[7][k] += tl + tr;
      }
    }
    if (tid == 0) P.split_on[i] = 1;
    __syncthreads();
  }

  // ---- 8. per-row gradient buckets (reduced over rows in a fixed order later)
  float* cr = P.contrib + (size_t)row * 8 * S;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int s = tid + k * NT;
      if (s < S) cr[(size_t)j * S + s] = c[j][k];
    }
}

#define KB_BWD_CASE(NT_, CPT_)                                                                   \
  if (S <= NT_ * CPT_) {                                                                         \
    hipLaunchKernelGGL((bwd_wave_kernel<NT_, CPT_>), dim3(W), dim3(NT_), 0, st, P, first);        \
    return;                                                                                      \
  }

void launch_bwd_wave(const BwdParams& P, int first, int W, hipStream_t st) {
  if (W <= 0) return;
  const int S = P.S;
  KB_BWD_CASE(64, 1)
  KB_BWD_CASE(128, 1)
  KB_BWD_CASE(256, 1)
  KB_BWD_CASE(256, 2)
  KB_BWD_CASE(512, 2)
  KB_BWD_CASE(512, 4)
  KB_BWD_CASE(1024, 4)
  KB_BWD_CASE(1024, 8)
}

// ---- backward constants from the saved tensors, in the glue's float32 order
// (_implicit_grad.py:136-143: DL = 1 + pD + E, SL1 = pS + E_s2, SL2 = pS + E_s1)
__global__ void bwd_consts_kernel(BwdConstArgs A) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= A.S) return;
  const float pS = A.log_pS[A.statewise ? s : 0];
  const float pD = A.log_pD[A.statewise ? s : 0];
  A.DL[s] = (1.0f + pD) + A.E[s];
  A.SL1[s] = pS + A.E_s2[s];
  A.SL2[s] = pS + A.E_s1[s];
  A.pS_state[s] = pS;
  A.pD_state[s] = pD;
}

void launch_bwd_consts(const BwdConstArgs& A, hipStream_t st) {
  hipLaunchKernelGGL(bwd_consts_kernel, dim3((A.S + 255) / 256), dim3(256), 0, st, A);
}

// ---- column sums of the per-row buckets over active rows, fixed order.
// Stage 1: chunk c of rows -> partial[c][8*S]; stage 2: sum of chunks.
constexpr int RED_CHUNK = 256;

__global__ void bwd_reduce_stage1(const float* contrib, const unsigned char* mask, int C, int S, double* partial) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;  // index in [0, 8S)
  const int chunk = blockIdx.y;
  if (j >= 8 * S) return;
  const int r0 = chunk * RED_CHUNK, r1 = min(C, r0 + RED_CHUNK);
  double acc = 0.0;
  for (int r = r0; r < r1; ++r)
    if (mask[r]) acc += (double)contrib[(size_t)r * 8 * S + j];
  partial[(size_t)chunk * 8 * S + j] = acc;
}

__global__ void bwd_reduce_stage2(const double* partial, int n_chunks, int S, double* out) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= 8 * S) return;
  double acc = 0.0;
  for (int c = 0; c < n_chunks; ++c) acc += partial[(size_t)c * 8 * S + j];
  out[j] = acc;
}

void launch_bwd_reduce(const float* contrib, const unsigned char* mask, int C, int S, double* partial,
                       double* out, hipStream_t st) {
  const int n_chunks = (C + RED_CHUNK - 1) / RED_CHUNK;
  dim3 g1((8 * S + 255) / 256, n_chunks);
  hipLaunchKernelGGL(bwd_reduce_stage1, g1, dim3(256), 0, st, contrib, mask, C, S, partial);
  hipLaunchKernelGGL(bwd_reduce_stage2, dim3((8 * S + 255) / 256), dim3(256), 0, st, partial, n_chunks, S, out);
}

int reduce_chunks(int C) { return (C + RED_CHUNK - 1) / RED_CHUNK; }

}  // namespace kb
