// Device helpers and host-side plumbing shared by the per-wrapper launchers
// (kb_ops.hip: primal kernels and their VJPs; kb_tangent.hip: forward
// tangents).  Internal to the library.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <map>
#include <mutex>
#include <utility>

#include "../../include/kbench_ops.h"
#include "kb_kernels.hpp"

namespace kbo {

constexpr int NT = 1024;
constexpr int NW = NT / 64;

struct OpsTree {
  int S, n_levels;
  const int* par;       // [S] parent column, -1 at the root
  const int* c1;        // [S] child columns, -1 if none
  const int* c2;
  const int* ev;        // [2S] Euler events: (column << 1) | is_exit
  const int* tin;       // [S] entry event of a column
  const int* pcol;      // [S] preorder position -> column
  const int* ppos;      // [S] column -> preorder position
  const int* pend;      // [S] column -> exclusive end of its subtree (preorder)
  const int* lvl_ptr;   // [n_levels + 1] depth levels, root level first
  const int* lvl_node;  // [S]
  const int* pc1;       // [S] preorder position -> position of child1, -1 if none
  const int* pc2;       // [S] preorder position -> position of child2, -1 if none
  const int* pnex;      // [S] preorder position i -> tin(column) - i, the postorder slots before entering i
  const int* ppost;     // [S] postorder slot -> preorder position (the order of the Euler exit events)
};

// ---- scalar helpers -------------------------------------------------------

template <typename T> __device__ __forceinline__ T ninf();
template <> __device__ __forceinline__ float ninf<float>() { return -__builtin_inff(); }
template <> __device__ __forceinline__ double ninf<double>() { return -__builtin_inf(); }

__device__ __forceinline__ float xexp2(float x) { return exp2f(x); }
__device__ __forceinline__ double xexp2(double x) { return exp2(x); }
__device__ __forceinline__ float xlog2(float x) { return log2f(x); }
__device__ __forceinline__ double xlog2(double x) { return log2(x); }

template <typename T>
__device__ __forceinline__ T msafe(T m) {
  return m == ninf<T>() ? T(0) : m;
}
template <typename T>
__device__ __forceinline__ T tmax(T a, T b) {
  return a > b ? a : b;
}

// Child column from a reference node_child array (a value outside [0, S): none).
__device__ __forceinline__ int child_at(const int64_t* c, int s, int S) {
  const int64_t v = c[s];
  return (v >= 0 && v < S) ? (int)v : -1;
}

// ---- block reductions and scans (generic, any T) ---------------------------

template <typename T>
__device__ __forceinline__ T wave_sum(T x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}
template <typename T>
__device__ __forceinline__ T wave_max(T x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = tmax(x, __shfl_xor(x, o, 64));
  return x;
}

// Both end with a barrier, so `red` may be reused right away.
template <typename T>
__device__ T block_sum(T x, T* red) {
  x = wave_sum(x);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  T t = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += red[i];
  __syncthreads();
  return t;
}
template <typename T>
__device__ T block_max(T x, T* red) {
  x = wave_max(x);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  T t = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) t = tmax(t, red[i]);
  __syncthreads();
  return t;
}

// In-place inclusive scan of a[0, n) in LDS; each thread scans a contiguous
// chunk.  Enters after the writers of a[] passed a barrier; ends with one.
template <typename T>
__device__ void block_scan(T* a, int n, T* red) {
  const int c = (n + NT - 1) / NT;
  const int b = min(n, (int)threadIdx.x * c), e = min(n, b + c);
  T s = 0;
  for (int i = b; i < e; ++i) s += a[i];
  T inc = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const T y = __shfl_up(inc, o, 64);
    if ((threadIdx.x & 63) >= (unsigned)o) inc += y;
  }
  if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = inc;
  __syncthreads();
  T run = inc - s;
  for (int w = 0; w < (int)(threadIdx.x >> 6); ++w) run += red[w];
  for (int i = b; i < e; ++i) {
    run += a[i];
    a[i] = run;
  }
  __syncthreads();
}

// Ancestors-or-self path sums: ps[s] = sum of x over the path root..s.  x and
// ps are LDS arrays in column order (ps may alias x); ev2 is LDS of 2S.
template <typename T>
__device__ void path_sums(const OpsTree& t, const T* x, T* ev2, T* ps, T* red) {
  const int S = t.S;
  for (int q = threadIdx.x; q < 2 * S; q += NT) {
    const int e = t.ev[q];
    const T v = x[e >> 1];
    ev2[q] = (e & 1) ? -v : v;
  }
  __syncthreads();
  block_scan(ev2, 2 * S, red);
  for (int s = threadIdx.x; s < S; s += NT) ps[s] = ev2[t.tin[s]];
  __syncthreads();
}

// Preorder prefix scan of u (column order, LDS) into pre[] (LDS, S); then
// the sum of u over the subtree of s is pre[pend[s]-1] - pre[ppos[s]-1] and
// over its complement pre[ppos[s]-1] + (total - pre[pend[s]-1]).
template <typename T>
__device__ void subtree_scan(const OpsTree& t, const T* u, T* pre, T* red) {
  for (int s = threadIdx.x; s < t.S; s += NT) pre[t.ppos[s]] = u[s];
  __syncthreads();
  block_scan(pre, t.S, red);
}
template <typename T>
__device__ __forceinline__ T subtree_of(const OpsTree& t, const T* pre, int s) {
  const int p = t.ppos[s], e = t.pend[s];
  return pre[e - 1] - (p > 0 ? pre[p - 1] : T(0));
}
template <typename T>
__device__ __forceinline__ T complement_of(const OpsTree& t, const T* pre, int s, T total) {
  const int p = t.ppos[s], e = t.pend[s];
  return (p > 0 ? pre[p - 1] : T(0)) + (total - pre[e - 1]);
}

// float64 path sums / subtree sums over depth levels (in place).
__device__ void level_path_sums(const OpsTree& t, double* x) {
  for (int d = 1; d < t.n_levels; ++d) {
    for (int i = t.lvl_ptr[d] + threadIdx.x; i < t.lvl_ptr[d + 1]; i += NT) {
      const int n = t.lvl_node[i];
      x[n] += x[t.par[n]];
    }
    __syncthreads();
  }
}
__device__ void level_subtree_sums(const OpsTree& t, double* x) {
  for (int d = t.n_levels - 2; d >= 0; --d) {
    for (int i = t.lvl_ptr[d] + threadIdx.x; i < t.lvl_ptr[d + 1]; i += NT) {
      const int n = t.lvl_node[i];
      double a = 0.0;
      if (t.c1[n] >= 0) a += x[t.c1[n]];
      if (t.c2[n] >= 0) a += x[t.c2[n]];
      x[n] += a;
    }
    __syncthreads();
  }
}

// Ancestors-or-self path sums of per-state register values x[k] (state
// threadIdx.x + k * NT): written as +x at the entry event and -x at the exit
// event of each column, scanned, read back at the entry event.  Enters with
// ev2 free; ends with a barrier after which ev2 may be reused.  V: the value
// type (double, or float for rows too long for three double rows of LDS).
template <int CPT, typename V>
__device__ void reg_path_sums(const OpsTree& t, const V (&x)[CPT], V (&ps)[CPT], V* ev2, V* red) {
  const int S = t.S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) {
      const int tin = t.tin[s];
      const int tout = tin + 2 * (t.pend[s] - t.ppos[s]) - 1;
      ev2[tin] = x[k];
      ev2[tout] = -x[k];
    }
  }
  __syncthreads();
  block_scan(ev2, 2 * S, red);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    ps[k] = s < S ? ev2[t.tin[s]] : V(0);
  }
  __syncthreads();
}

// Subtree-or-self sums of per-state register values x[k]: x scattered to
// preorder positions, scanned, differenced over each subtree's range.
// Enters with buf (S values) free; ends with a barrier.
template <int CPT, typename V>
__device__ void reg_subtree_sums(const OpsTree& t, const V (&x)[CPT], V (&sub)[CPT], V* buf, V* red) {
  const int S = t.S;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    if (s < S) buf[t.ppos[s]] = x[k];
  }
  __syncthreads();
  block_scan(buf, S, red);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int s = threadIdx.x + k * NT;
    sub[k] = V(0);
    if (s < S) {
      const int p = t.ppos[s], e = t.pend[s];
      sub[k] = buf[e - 1] - (p > 0 ? buf[p - 1] : V(0));
    }
  }
  __syncthreads();
}

}  // namespace kbo

// =====================================================================================
// host side
// =====================================================================================

struct kb_tree {
  int S = 0, n_levels = 0;
  int *par = nullptr, *c1 = nullptr, *c2 = nullptr, *ev = nullptr, *tin = nullptr;
  int *pcol = nullptr, *ppos = nullptr, *pend = nullptr, *lvl_ptr = nullptr, *lvl_node = nullptr;
  int *pc1 = nullptr, *pc2 = nullptr, *pnex = nullptr, *ppost = nullptr;
  kbo::OpsTree dev() const {
    return kbo::OpsTree{S, n_levels, par, c1, c2, ev, tin, pcol, ppos, pend, lvl_ptr, lvl_node,
                        pc1, pc2, pnex, ppost};
  }
};

namespace kbo_host {

#define KBO_HIP(expr)                                                                      \
  do {                                                                                     \
    hipError_t _e = (expr);                                                                \
    if (_e != hipSuccess) return kb::set_error(KB_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

constexpr size_t LDS_BYTES = 160 * 1024 - 2048;  // minus the static reduction arrays

inline int cpt_for(int S) {
  if (S <= 1024) return 1;
  if (S <= 2048) return 2;
  if (S <= 4096) return 4;
  if (S <= 8192) return 8;
  return 0;
}

inline size_t elem_size(int dtype) { return dtype == KB_F64 ? 8 : (dtype == KB_BF16 ? 2 : 4); }

inline int check_lds(size_t bytes, int S, int dtype) {
  if (bytes > LDS_BYTES)
    return kb::set_error(KB_ERR_ARG, "S=%d needs %zu bytes of LDS per row for dtype %s (limit %zu)", S, bytes,
                         dtype == KB_F64 ? "float64" : "float32", LDS_BYTES);
  return 0;
}

// LDS of the kernels that keep three rows of S (a row and a 2S scan buffer):
// float64 arithmetic while three float64 rows fit, float32 arithmetic in three
// float32 rows for longer float32 rows (they need CPT = 8), an error for
// longer float64 rows.
inline int three_row_lds(int S, int dtype, size_t* lds, bool* f32) {
  const size_t b64 = (size_t)3 * S * sizeof(double);
  *f32 = dtype == KB_F32 && b64 > LDS_BYTES;
  *lds = *f32 ? (size_t)3 * S * sizeof(float) : b64;
  return check_lds(*lds, S, *f32 ? KB_F32 : KB_F64);
}

inline hipStream_t st_of(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int dtype_ok(int dtype) {
  if (dtype != KB_F32 && dtype != KB_F64) return kb::set_error(KB_ERR_ARG, "dtype must be float32 or float64");
  return 0;
}

// Dispatch a kernel template over (T, CPT).
#define KBO_DISPATCH(DTYPE, S, ...)                                         \
  do {                                                                       \
    const int _cpt = cpt_for(S);                                             \
    if (_cpt == 0) return kb::set_error(KB_ERR_ARG, "S=%d exceeds 8192", S); \
    if ((DTYPE) == KB_F64) {                                                 \
      using T = double;                                                      \
      switch (_cpt) {                                                        \
        case 1: { constexpr int CPT = 1; __VA_ARGS__; } break;                      \
        case 2: { constexpr int CPT = 2; __VA_ARGS__; } break;                      \
        case 4: { constexpr int CPT = 4; __VA_ARGS__; } break;                      \
        default: { constexpr int CPT = 8; __VA_ARGS__; } break;                     \
      }                                                                      \
    } else {                                                                 \
      using T = float;                                                       \
      switch (_cpt) {                                                        \
        case 1: { constexpr int CPT = 1; __VA_ARGS__; } break;                      \
        case 2: { constexpr int CPT = 2; __VA_ARGS__; } break;                      \
        case 4: { constexpr int CPT = 4; __VA_ARGS__; } break;                      \
        default: { constexpr int CPT = 8; __VA_ARGS__; } break;                     \
      }                                                                      \
    }                                                                        \
  } while (0)

// Raise a kernel's dynamic-LDS limit to what this launch needs.  The limit set
// so far is remembered per kernel and device, so a launch at or below it makes
// no runtime call (the per-call wrappers launch thousands of times per solve).
template <typename F>
inline int set_lds(F* kernel, size_t bytes) {
  if (bytes <= 64 * 1024) return 0;
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> raised;
  int dev = 0;
  KBO_HIP(hipGetDevice(&dev));
  const auto key = std::make_pair(reinterpret_cast<const void*>(kernel), dev);
  std::lock_guard<std::mutex> lock(mu);
  auto it = raised.find(key);
  if (it != raised.end() && it->second >= bytes) return 0;
  KBO_HIP(hipFuncSetAttribute(key.first, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
  raised[key] = bytes;
  return 0;
}

}  // namespace kbo_host
