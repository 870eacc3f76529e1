// Device-side building blocks shared by every kernel of the solver path.
//
// Conventions:
//  * one workgroup owns one clade row of S state columns; thread t owns the
//    columns t, t + NT, t + 2*NT, ... (so row loads and stores are coalesced);
//  * the species tree is held as int32 tables with -1 meaning "no node";
//  * path sums over ancestors-or-self use pointer jumping: jump[t][s] is the
//    2^t-th ancestor of s (or -1), so ceil(log2(max_depth)) LDS rounds replace
//    the reference's per-column walk of max_ancestor_depth dependent gathers;
//  * subtree sums (the transpose of the path sum) run bottom-up over internal
//    nodes grouped by depth, deepest level first.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define KB_NEG_INF (-__builtin_inff())
#define KB_MAX_JUMP 16

namespace kb {

struct TreeDev {
  int S;
  int n_jump;                 // number of pointer-jumping rounds
  int n_blevels;              // bottom-up levels (internal nodes)
  const int* parent;          // [S]
  const int* c1;              // [S] (-1: none)
  const int* c2;              // [S]
  const int* jump;            // [n_jump, S]
  const int* blevel_ptr;      // [n_blevels + 1]
  const int* blevel_node;     // [n_internal] deepest level first
  const int* sub_start;       // [S] preorder index
  const int* sub_end;         // [S] preorder index + subtree size
};

__device__ __forceinline__ float fsafe(float m) { return m == KB_NEG_INF ? 0.0f : m; }

// 2^x by the hardware instruction: the same as exp2f for x >= -126 and 0 below
// (where exp2f returns a denormal).  For terms whose size next to the others
// of their sum or product makes such values negligible.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// log2 x by the hardware instruction: the same as log2f for x >= 2^-126 and
// for 0; for the sums of max-shifted terms, which are 0 or at least 1.
__device__ __forceinline__ float log2_hw(float x) { return __builtin_amdgcn_logf(x); }

// 1/x by the hardware reciprocal (1 ulp) instead of a correctly rounded division.
__device__ __forceinline__ float rcp_hw(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ double dsafe(double m) { return m == -__builtin_inf() ? 0.0 : m; }

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    T u = __shfl_xor(v, o, 64);
    v = u > v ? u : v;
  }
  return v;
}

// Block-wide reductions. `red` is LDS scratch of at least NT/64 elements.
// Every thread returns the full result. Two barriers (reuse-safe).
template <int NT, typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
  constexpr int NW = NT / 64;
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  T r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r += red[i];
  __syncthreads();
  return r;
}

template <int NT, typename T>
__device__ __forceinline__ T block_max(T v, T* red) {
  constexpr int NW = NT / 64;
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  T r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = red[i] > r ? red[i] : r;
  __syncthreads();
  return r;
}

// ---- float64 tree sums by prefix scans (depth-independent) -------------------
// Preorder and Euler-tour tables in column terms: every subtree is the
// preorder range [pre(s), endpos[pre(s)]); the Euler tour lists (column << 1)
// on entry and (column << 1) | 1 on exit, tin_col[s] is the entry event.
struct TreeScanDev {
  int S;
  const int* pre;        // [S] column -> preorder position
  const int* endpos;     // [S] position -> exclusive end of its subtree
  const int* euler_col;  // [2S]
  const int* tin_col;    // [S]
};

// In-place inclusive scan of a[0, n) (LDS); contiguous chunk per thread.
// The writers of a[] must have passed a barrier; ends with a barrier.
template <int NT>
__device__ void scan_incl_f64(double* a, int n, double* red) {
  const int c = (n + NT - 1) / NT;
  const int b = min(n, (int)threadIdx.x * c), e = min(n, b + c);
  double s = 0.0;
  for (int i = b; i < e; ++i) s += a[i];
  double inc = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double y = __shfl_up(inc, o, 64);
    if ((int)(threadIdx.x & 63) >= o) inc += y;
  }
  if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = inc;
  __syncthreads();
  double run = inc - s;
  for (int w = 0; w < (int)(threadIdx.x >> 6); ++w) run += red[w];
  for (int i = b; i < e; ++i) {
    run += a[i];
    a[i] = run;
  }
  __syncthreads();
}

// Ancestors-or-self path sums of x[] in place (column order, LDS, published);
// scan2: LDS scratch of 2S doubles.
template <int NT>
__device__ void euler_path_sums_f64(const TreeScanDev& t, double* x, double* scan2, double* red) {
  const int S = t.S;
  for (int q = threadIdx.x; q < 2 * S; q += NT) {
    const int e = t.euler_col[q];
    const double v = x[e >> 1];
    scan2[q] = (e & 1) ? -v : v;
  }
  __syncthreads();
  scan_incl_f64<NT>(scan2, 2 * S, red);
  for (int s = threadIdx.x; s < S; s += NT) x[s] = scan2[t.tin_col[s]];
  __syncthreads();
}

// Descendants-or-self (subtree) sums of u[] in place (column order, LDS,
// published); tmp: LDS scratch of S doubles.
template <int NT>
__device__ void preorder_subtree_sums_f64(const TreeScanDev& t, double* u, double* tmp, double* red) {
  const int S = t.S;
  for (int s = threadIdx.x; s < S; s += NT) tmp[t.pre[s]] = u[s];
  __syncthreads();
  scan_incl_f64<NT>(tmp, S, red);
  for (int s = threadIdx.x; s < S; s += NT) {
    const int p = t.pre[s], e = t.endpos[p];
    u[s] = tmp[e - 1] - (p > 0 ? tmp[p - 1] : 0.0);
  }
  __syncthreads();
}

// Ancestors-or-self path sums of `val` (already in LDS buffer a[]).
// Uses a[] and b[] as ping-pong buffers; returns the buffer holding the result.
// Caller must __syncthreads() after writing a[] and before calling.
template <int NT, int CPT, typename T>
__device__ __forceinline__ T* path_sum_lds(const TreeDev& tr, T* a, T* b) {
  T* src = a;
  T* dst = b;
  for (int t = 0; t < tr.n_jump; ++t) {
    const int* jt = tr.jump + (size_t)t * tr.S;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      int s = threadIdx.x + k * NT;
      if (s < tr.S) {
        int j = jt[s];
        dst[s] = src[s] + (j >= 0 ? src[j] : T(0));
      }
    }
    __syncthreads();
    T* tmp = src;
    src = dst;
    dst = tmp;
  }
  return src;
}

// In-place bottom-up subtree sums of the LDS vector u[] (internal nodes by
// depth, deepest level first). Caller syncs before; ends synced.
template <int NT, typename T>
__device__ __forceinline__ void subtree_sum_lds(const TreeDev& tr, T* u) {
  for (int lv = 0; lv < tr.n_blevels; ++lv) {
    const int b = tr.blevel_ptr[lv], e = tr.blevel_ptr[lv + 1];
    for (int i = b + threadIdx.x; i < e; i += NT) {
      int p = tr.blevel_node[i];
      int x = tr.c1[p], y = tr.c2[p];
      T add = (x >= 0 ? u[x] : T(0)) + (y >= 0 ? u[y] : T(0));
      u[p] += add;
    }
    __syncthreads();
  }
}

// log2-sum-exp2 of up to 7 float terms, reference order: max, m_safe, sum, log2 + m.
__device__ __forceinline__ float lse2_5(float t0, float t1, float t2, float t3, float t4) {
  float m = fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), t4);
  float ms = fsafe(m);
  float s = exp2f(t0 - ms) + exp2f(t1 - ms) + exp2f(t2 - ms) + exp2f(t3 - ms) + exp2f(t4 - ms);
  return log2f(s) + m;
}

// Online merge of a (max, scaled-sum) pair into an accumulator.
__device__ __forceinline__ void lse_merge(float& m, float& acc, float m2, float s2) {
  float nm = fmaxf(m, m2);
  float nms = fsafe(nm);
  float a = (m == KB_NEG_INF) ? 0.0f : acc * exp2_hw(m - nms);
  float b = (m2 == KB_NEG_INF) ? 0.0f : s2 * exp2_hw(m2 - nms);
  acc = a + b;
  m = nm;
}

// Rate parameter addressing of the split terms (reference dts_fused.py:11-15).
struct RateDev {
  const float* p;
  int row_stride;   // 0 when the parameter has a single row
  int by_state;     // per-column values
  __device__ __forceinline__ float at(int item, int s) const {
    return by_state ? p[(size_t)item * row_stride + s] : p[(size_t)item * row_stride];
  }
};

}  // namespace kb
