// Row operations in preorder, wavefront-segment ownership.
//
// Inside a row kernel with NT threads (NW = NT/64 wavefronts), wavefront w owns
// the preorder segment [w*SEG, (w+1)*SEG), SEG = 64*CPT, and lane l of it owns
// positions w*SEG + k*64 + l for k < CPT ("slot k").  For a fixed slot the 64
// lanes touch 64 consecutive positions, so LDS reads/writes of own positions
// are bank-conflict free, and the position order is (wave, slot, lane).
//
// In preorder every subtree is a contiguous range [i, end(i)), so
//   * the sum over the complement of a subtree (the transpose of the
//     "all non-ancestors" sum) is  scan[i-1] + (total - scan[end(i)-1])  for an
//     inclusive prefix scan over positions;
//   * the ancestors-or-self path sum of node i is the prefix, up to i's entry,
//     of its Euler tour (+x on entry, -x on exit).
// Both are one block scan: DPP row shifts / row broadcasts inside a wavefront,
// a running carry across slots, and one LDS exchange of wavefront totals.
#pragma once

#include "kb_device.hpp"

namespace kb {

// ---- wavefront primitives (DPP) ---------------------------------------------

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp_shift0(float x) {
  // lanes without a source read 0 (the identity of +)
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, BANK_MASK, false));
}

// Inclusive scan (+) across the 64 lanes of a wavefront.
__device__ __forceinline__ float wave_scan_incl(float x) {
  x += dpp_shift0<0x111>(x);       // row_shr:1
  x += dpp_shift0<0x112>(x);       // row_shr:2
  x += dpp_shift0<0x114>(x);       // row_shr:4
  x += dpp_shift0<0x118>(x);       // row_shr:8
  x += dpp_shift0<0x142, 0xa>(x);  // row_bcast:15 -> rows 1, 3
  x += dpp_shift0<0x143, 0xc>(x);  // row_bcast:31 -> rows 2, 3
  return x;
}

// Value of the previous lane (lane 0 reads 0): DPP wavefront shift.
__device__ __forceinline__ float wave_prev_lane(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x138, 0xf, 0xf, false));  // wave_shr:1
}

// Per-wavefront values published in LDS (w[0..NW-1]), read by lanes 0..NW-1
// (zero elsewhere) without a branch, so the scheduler can issue the read
// together with the gathers around it.  NW is a power of two.
template <int NW, typename T>
__device__ __forceinline__ T lds_wave_values(const T* w, int lane, T zero) {
  static_assert((NW & (NW - 1)) == 0, "power of two");
  const T x = w[lane & (NW - 1)];
  return lane < NW ? x : zero;
}

// Inclusive scan (+) over lanes [0, N) of a wavefront, N <= 16 (row 0 only;
// the other lanes hold partial sums).
template <int N>
__device__ __forceinline__ float wave_scan_first(float x) {
  static_assert(N >= 1 && N <= 16, "row-0 scan");
  if constexpr (N > 1) x += dpp_shift0<0x111>(x);
  if constexpr (N > 2) x += dpp_shift0<0x112>(x);
  if constexpr (N > 4) x += dpp_shift0<0x114>(x);
  if constexpr (N > 8) x += dpp_shift0<0x118>(x);
  return x;
}

__device__ __forceinline__ float lane_value(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

__device__ __forceinline__ float wave_reduce_sum(float x) { return lane_value(wave_scan_incl(x), 63); }

__device__ __forceinline__ float wave_reduce_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}

// ---- global accesses of the large-row kernels ----------------------------------

// b[i] through a 32-bit byte offset from a uniform base.
template <typename T>
__device__ __forceinline__ T ldg(const T* b, int i) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(b) + (unsigned)i * (unsigned)sizeof(T));
}
template <typename T>
__device__ __forceinline__ void stg(T* b, int i, T x) {
  *reinterpret_cast<T*>(reinterpret_cast<char*>(b) + (unsigned)i * (unsigned)sizeof(T)) = x;
}

// The same uniform pointer, opaque to the optimiser for each value of
// `epoch`.  A kernel passes a different epoch in each phase or iteration (the
// row and phase, the split, the sweep), so the per-lane addresses of its
// tables are formed where they are used: with plain pointers they are computed
// once and hoisted out of the loops, held in register pairs across them.  The
// asm has no side effects, so loads around it still issue together.
template <typename T>
__device__ __forceinline__ T* fresh(T* p, int epoch) {
  unsigned long long x = reinterpret_cast<unsigned long long>(p);
  asm("; %1" : "+s"(x) : "s"(epoch));
  // a global-memory pointer again, so the accesses stay global (not flat)
  return (T*)reinterpret_cast<__attribute__((address_space(1))) T*>(x);
}

// ---- float64 wavefront primitives (DPP on the two 32-bit halves) -------------

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ double dpp_shift0_f64(double x) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(x);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, ROW_MASK, BANK_MASK, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, ROW_MASK, BANK_MASK, false);
  return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}

__device__ __forceinline__ double wave_scan_incl_f64(double x) {
  x += dpp_shift0_f64<0x111>(x);
  x += dpp_shift0_f64<0x112>(x);
  x += dpp_shift0_f64<0x114>(x);
  x += dpp_shift0_f64<0x118>(x);
  x += dpp_shift0_f64<0x142, 0xa>(x);
  x += dpp_shift0_f64<0x143, 0xc>(x);
  return x;
}

template <int N>
__device__ __forceinline__ double wave_scan_first_f64(double x) {
  static_assert(N >= 1 && N <= 16, "row-0 scan");
  if constexpr (N > 1) x += dpp_shift0_f64<0x111>(x);
  if constexpr (N > 2) x += dpp_shift0_f64<0x112>(x);
  if constexpr (N > 4) x += dpp_shift0_f64<0x114>(x);
  if constexpr (N > 8) x += dpp_shift0_f64<0x118>(x);
  return x;
}

__device__ __forceinline__ double lane_value_f64(double x, int lane) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(x);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, lane);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), lane);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

__device__ __forceinline__ double wave_prev_lane_f64(double x) { return dpp_shift0_f64<0x138>(x); }  // wave_shr:1

__device__ __forceinline__ double shfl_f64(double x, int src) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(x);
  const unsigned lo = (unsigned)__shfl((int)(unsigned)b, src, 64);
  const unsigned hi = (unsigned)__shfl((int)(unsigned)(b >> 32), src, 64);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Own positions (contiguous ownership) of a float64 LDS row.
template <int CPT>
__device__ __forceinline__ void lds_store_own_f64(double* lds, const double (&v)[CPT]) {
  double* p = lds + threadIdx.x * CPT;
  if constexpr (CPT % 2 == 0) {
#pragma unroll
    for (int k = 0; k < CPT; k += 2) *reinterpret_cast<double2*>(p + k) = make_double2(v[k], v[k + 1]);
  } else {
#pragma unroll
    for (int k = 0; k < CPT; ++k) p[k] = v[k];
  }
}

// ---- block reductions / scans (one barrier each) -----------------------------
// `wtot` is LDS scratch of NW floats (2*NW for the paired scan).  It is read
// by every thread after the barrier, so the next writer must be separated from
// these reads by another barrier: callers alternate scratch arrays.

template <int NT>
__device__ __forceinline__ float block_sum1(float x, float* wtot) {
  constexpr int NW = NT / 64;
  const float ws = wave_reduce_sum(x);
  if ((threadIdx.x & 63) == 0) wtot[threadIdx.x >> 6] = ws;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += wtot[i];
  return t;
}

template <int NT>
__device__ __forceinline__ float block_max1(float x, float* wtot) {
  constexpr int NW = NT / 64;
  const float wm = wave_reduce_max(x);
  if ((threadIdx.x & 63) == 0) wtot[threadIdx.x >> 6] = wm;
  __syncthreads();
  float t = KB_NEG_INF;
#pragma unroll
  for (int i = 0; i < NW; ++i) t = fmaxf(t, wtot[i]);
  return t;
}

// In-place inclusive scan over positions of v[k] (slot k of this lane).
// Returns the block total.
template <int NT, int N>
__device__ __forceinline__ float block_scan_incl(float (&v)[N], float* wtot) {
  constexpr int NW = NT / 64;
  float carry = 0.0f;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const float s = wave_scan_incl(v[k]);
    v[k] = s + carry;
    carry += lane_value(s, 63);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) wtot[w] = carry;
  __syncthreads();
  float off = 0.0f, total = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const float t = wtot[i];
    if (i < w) off += t;
    total += t;
  }
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] += off;
  return total;
}

// Two scans sharing one barrier (wtot holds 2*NW floats).
template <int NT, int N>
__device__ __forceinline__ void block_scan_incl2(float (&a)[N], float (&b)[N], float* wtot, float& ta, float& tb) {
  constexpr int NW = NT / 64;
  float ca = 0.0f, cb = 0.0f;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const float sa = wave_scan_incl(a[k]);
    const float sb = wave_scan_incl(b[k]);
    a[k] = sa + ca;
    b[k] = sb + cb;
    ca += lane_value(sa, 63);
    cb += lane_value(sb, 63);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    wtot[w] = ca;
    wtot[NW + w] = cb;
  }
  __syncthreads();
  float oa = 0.0f, ob = 0.0f;
  ta = 0.0f;
  tb = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const float x = wtot[i], y = wtot[NW + i];
    if (i < w) {
      oa += x;
      ob += y;
    }
    ta += x;
    tb += y;
  }
#pragma unroll
  for (int k = 0; k < N; ++k) {
    a[k] += oa;
    b[k] += ob;
  }
}

// ---- preorder tables ---------------------------------------------------------

struct PreDev {
  int S;
  const int* pre;     // [S]   column -> preorder position
  const int* col;     // [S]   position -> column
  const int* c1pos;   // [S]   position of node_child1 (-1: leaf)
  const int* c2pos;   // [S]   position of node_child2 (-1: leaf)
  const int* ppos;    // [S]   position of the parent (-1: root)
  const int* pflag;   // [S]   1 if this position is node_child1 of its parent
  const int* endpos;  // [S]   exclusive end of the subtree
  const int* tin;     // [S]   Euler entry event of the position
  const int* euler;   // [2S]  event -> (position << 1) | is_exit
  const int* post;    // [S]   postorder slot -> position (the order of the Euler exit events)
};

// Position of slot k of this thread.
template <int NT, int CPT>
__device__ __forceinline__ int own_pos(int k) {
  return (threadIdx.x >> 6) * (64 * CPT) + k * 64 + (threadIdx.x & 63);
}

// Euler event of slot j (< 2*CPT) of this thread.
template <int NT, int CPT>
__device__ __forceinline__ int own_event(int j) {
  return (threadIdx.x >> 6) * (128 * CPT) + j * 64 + (threadIdx.x & 63);
}

// Per-thread copy of the preorder tables of its own positions and events.
// Invalid entries point at the padding slot ZERO (= NT*CPT) of the LDS row
// buffers, which always holds 0, so the sweep loops need no bounds branches.
// Euler events are owned contiguously: thread t holds events
// [t*2*CPT, (t+1)*2*CPT), so their scan is a sequential local scan plus one
// wavefront scan.
template <int NT, int CPT>
struct OwnTables {
  static constexpr int ZERO = NT * CPT;
  int col[CPT], c1p[CPT], c2p[CPT], tin[CPT];
  int ev[2 * CPT];  // (position << 1) | is_exit; padding: ZERO << 1
  __device__ __forceinline__ void load(const PreDev& T) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int i = own_pos<NT, CPT>(k);
      const bool ok = i < T.S;
      col[k] = ok ? T.col[i] : -1;
      const int a = ok ? T.c1pos[i] : -1, b = ok ? T.c2pos[i] : -1;
      c1p[k] = a >= 0 ? a : ZERO;
      c2p[k] = b >= 0 ? b : ZERO;
      tin[k] = ok ? T.tin[i] : 0;
    }
#pragma unroll
    for (int j = 0; j < 2 * CPT; ++j) {
      const int q = threadIdx.x * (2 * CPT) + j;
      ev[j] = q < 2 * T.S ? T.euler[q] : (ZERO << 1);
    }
  }
};

// ---- contiguous ownership ------------------------------------------------------
// Alternative layout for kernels whose inner loop is a block scan: thread t owns
// positions t*CPT + k, so a scan is a per-thread running sum plus ONE wavefront
// scan of the thread totals (instead of one per slot), and the scan value at
// position i-1 of slot 0 is the previous lane's last value.  Own positions are
// moved to and from LDS with vector accesses (conflict-free).

// Minimum waves per SIMD asked of the 1024-thread preorder-ownership sweep and
// adjoint kernels: eight (two resident workgroups per CU, at most 64 VGPRs)
// when a thread owns at most two positions, else no constraint.
constexpr int pre_waves_per_eu(int cpt) { return cpt <= 2 ? 8 : 1; }

template <int NT, int CPT>
__device__ __forceinline__ int own_pos_c(int k) {
  return threadIdx.x * CPT + k;
}

// Own positions t*CPT .. t*CPT+CPT-1 of a global row p[0..n): one vector load
// (16 bytes per four positions, 8 bytes for two) where all of them are below
// n, else element by element with `fill` past n.  p must be 16-byte aligned
// (every row these read starts its own allocation or a multiple of four
// elements into one), so the vector accesses never cross the row's end.
template <int CPT, typename T>
__device__ __forceinline__ void gld_own(const T* p, int n, T (&v)[CPT], T fill) {
  static_assert(sizeof(T) == 4, "32-bit elements");
  const int b = threadIdx.x * CPT;
  if (b + CPT <= n) {
    if constexpr (CPT % 4 == 0) {
#pragma unroll
      for (int k = 0; k < CPT; k += 4) {
        const int4 q = *reinterpret_cast<const int4*>(p + b + k);
        v[k] = __builtin_bit_cast(T, q.x);
        v[k + 1] = __builtin_bit_cast(T, q.y);
        v[k + 2] = __builtin_bit_cast(T, q.z);
        v[k + 3] = __builtin_bit_cast(T, q.w);
      }
    } else if constexpr (CPT % 2 == 0) {
#pragma unroll
      for (int k = 0; k < CPT; k += 2) {
        const int2 q = *reinterpret_cast<const int2*>(p + b + k);
        v[k] = __builtin_bit_cast(T, q.x);
        v[k + 1] = __builtin_bit_cast(T, q.y);
      }
    } else {
#pragma unroll
      for (int k = 0; k < CPT; ++k) v[k] = p[b + k];
    }
  } else {
#pragma unroll
    for (int k = 0; k < CPT; ++k) v[k] = b + k < n ? p[b + k] : fill;
  }
}

// The store counterpart of gld_own: positions at or past n are not written.
template <int CPT>
__device__ __forceinline__ void gst_own(float* p, int n, const float (&v)[CPT]) {
  const int b = threadIdx.x * CPT;
  if (b + CPT <= n) {
    if constexpr (CPT % 4 == 0) {
#pragma unroll
      for (int k = 0; k < CPT; k += 4)
        *reinterpret_cast<float4*>(p + b + k) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
    } else if constexpr (CPT % 2 == 0) {
#pragma unroll
      for (int k = 0; k < CPT; k += 2) *reinterpret_cast<float2*>(p + b + k) = make_float2(v[k], v[k + 1]);
    } else {
#pragma unroll
      for (int k = 0; k < CPT; ++k) p[b + k] = v[k];
    }
  } else {
#pragma unroll
    for (int k = 0; k < CPT; ++k)
      if (b + k < n) p[b + k] = v[k];
  }
}

template <int CPT>
__device__ __forceinline__ void lds_store_own(float* lds, const float (&v)[CPT]) {
  float* p = lds + threadIdx.x * CPT;
  if constexpr (CPT % 4 == 0) {
#pragma unroll
    for (int k = 0; k < CPT; k += 4) *reinterpret_cast<float4*>(p + k) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
  } else if constexpr (CPT % 2 == 0) {
#pragma unroll
    for (int k = 0; k < CPT; k += 2) *reinterpret_cast<float2*>(p + k) = make_float2(v[k], v[k + 1]);
  } else {
#pragma unroll
    for (int k = 0; k < CPT; ++k) p[k] = v[k];
  }
}

template <int CPT>
__device__ __forceinline__ void lds_load_own(const float* lds, float (&v)[CPT]) {
  const float* p = lds + threadIdx.x * CPT;
  if constexpr (CPT % 4 == 0) {
#pragma unroll
    for (int k = 0; k < CPT; k += 4) {
      const float4 q = *reinterpret_cast<const float4*>(p + k);
      v[k] = q.x;
      v[k + 1] = q.y;
      v[k + 2] = q.z;
      v[k + 3] = q.w;
    }
  } else if constexpr (CPT % 2 == 0) {
#pragma unroll
    for (int k = 0; k < CPT; k += 2) {
      const float2 q = *reinterpret_cast<const float2*>(p + k);
      v[k] = q.x;
      v[k + 1] = q.y;
    }
  } else {
#pragma unroll
    for (int k = 0; k < CPT; ++k) v[k] = p[k];
  }
}

// In-place inclusive scan over positions of contiguously owned v[]; returns the
// block total.  One barrier; callers alternate `wtot` arrays.
template <int NT, int CPT>
__device__ __forceinline__ float block_scan_incl_c(float (&v)[CPT], float* wtot) {
  constexpr int NW = NT / 64;
#pragma unroll
  for (int k = 1; k < CPT; ++k) v[k] += v[k - 1];
  const float tsum = v[CPT - 1];
  const float ws = wave_scan_incl(tsum);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 63) wtot[w] = ws;
  __syncthreads();
  float off = ws - tsum, total = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const float t = wtot[i];
    if (i < w) off += t;
    total += t;
  }
#pragma unroll
  for (int k = 0; k < CPT; ++k) v[k] += off;
  return total;
}

// Subtree sums with one barrier.  Before it, local_scan_publish stores the
// wavefront-local inclusive scan of u (own positions) at L and the wavefront
// total at wt[wavefront]; after it, subtree_terms gives for every own
// position i  P(i - 1)  and  A - P(end(i) - 1)  of the block-wide inclusive
// scan P (A its total, P(-1) = 0), adding the wavefront offsets to what it
// reads.  wend[k] is the wavefront that owns end(i) - 1.
template <int NT, int CPT>
__device__ __forceinline__ void local_scan_publish(float (&sc)[CPT], const float (&u)[CPT], float* L, float* wt) {
  float t = 0.0f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    t += u[k];
    sc[k] = t;
  }
  const float ws = wave_scan_incl(t);
  if ((threadIdx.x & 63) == 63) wt[threadIdx.x >> 6] = ws;
#pragma unroll
  for (int k = 0; k < CPT; ++k) sc[k] += ws - t;
  lds_store_own<CPT>(L, sc);
}

template <int NT, int CPT>
__device__ __forceinline__ void subtree_terms(const float (&sc)[CPT], const float* L, const float* wt,
                                              const int (&endm1)[CPT], const int (&wend)[CPT], float (&pm1)[CPT],
                                              float (&rest)[CPT]) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  float le[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) le[k] = L[endm1[k]];
  const float wtot = lds_wave_values<NW>(wt, lane, 0.0f);
  const float wincl = wave_scan_first<NW>(wtot);
  const float wexcl = wincl - wtot;  // lane x < NW: offset of wavefront x
  const float A = lane_value(wincl, NW - 1);
  const float woff = lane_value(wexcl, wv);
  const float p0 = wave_prev_lane(sc[CPT - 1]) + woff;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    pm1[k] = k == 0 ? p0 : sc[k - 1] + woff;
    rest[k] = A - (le[k] + __shfl(wexcl, wend[k], 64));
  }
}

// Two contiguous-ownership scans sharing one barrier (wtot holds 2*NW floats).
template <int NT, int CPT>
__device__ __forceinline__ void block_scan_incl2_c(float (&a)[CPT], float (&b)[CPT], float* wtot, float& ta,
                                                   float& tb) {
  constexpr int NW = NT / 64;
#pragma unroll
  for (int k = 1; k < CPT; ++k) {
    a[k] += a[k - 1];
    b[k] += b[k - 1];
  }
  const float sa = a[CPT - 1], sb = b[CPT - 1];
  const float wa = wave_scan_incl(sa), wb = wave_scan_incl(sb);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 63) {
    wtot[w] = wa;
    wtot[NW + w] = wb;
  }
  __syncthreads();
  float oa = wa - sa, ob = wb - sb;
  ta = 0.0f;
  tb = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const float x = wtot[i], y = wtot[NW + i];
    if (i < w) {
      oa += x;
      ob += y;
    }
    ta += x;
    tb += y;
  }
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    a[k] += oa;
    b[k] += ob;
  }
}

// Preorder tables of the contiguously owned positions (same fields as
// OwnTables; the Euler events are owned contiguously in both layouts).
template <int NT, int CPT>
struct OwnTablesC {
  static constexpr int ZERO = NT * CPT;
  int col[CPT], c1p[CPT], c2p[CPT], tin[CPT];
  int ev[2 * CPT];
  // VEC: one vector load per table (fewer memory instructions in flight, more
  // registers live at once); else one load per position
  template <bool VEC = false>
  __device__ __forceinline__ void load(const PreDev& T) {
    if constexpr (VEC) {
      int a[CPT], b[CPT];
      gld_own<CPT>(T.col, T.S, col, -1);
      gld_own<CPT>(T.c1pos, T.S, a, -1);
      gld_own<CPT>(T.c2pos, T.S, b, -1);
      gld_own<CPT>(T.tin, T.S, tin, 0);
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        c1p[k] = a[k] >= 0 ? a[k] : ZERO;
        c2p[k] = b[k] >= 0 ? b[k] : ZERO;
      }
      gld_own<2 * CPT>(T.euler, 2 * T.S, ev, ZERO << 1);
    } else {
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int i = own_pos_c<NT, CPT>(k);
        const bool ok = i < T.S;
        col[k] = ok ? T.col[i] : -1;
        const int a = ok ? T.c1pos[i] : -1, b = ok ? T.c2pos[i] : -1;
        c1p[k] = a >= 0 ? a : ZERO;
        c2p[k] = b >= 0 ? b : ZERO;
        tin[k] = ok ? T.tin[i] : 0;
      }
#pragma unroll
      for (int j = 0; j < 2 * CPT; ++j) {
        const int q = threadIdx.x * (2 * CPT) + j;
        ev[j] = q < 2 * T.S ? T.euler[q] : (ZERO << 1);
      }
    }
  }
};

// Coalesced load of a global row (column order) into LDS at preorder
// positions, then into v[] (own positions).  One barrier; the caller separates
// reuse of `lds` with a barrier.  Positions >= S read `fill`.
template <int NT, int CPT>
__device__ __forceinline__ void load_row_pre(const PreDev& T, const float* grow, float* lds, float (&v)[CPT],
                                             float fill) {
  for (int s = threadIdx.x; s < T.S; s += NT) lds[T.pre[s]] = grow[s];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = own_pos<NT, CPT>(k);
    v[k] = i < T.S ? lds[i] : fill;
  }
}

// Own positions -> LDS -> coalesced global row in column order.  One barrier.
template <int NT, int CPT>
__device__ __forceinline__ void store_row_pre(const PreDev& T, const float (&v)[CPT], float* lds, float* grow) {
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int i = own_pos<NT, CPT>(k);
    if (i < T.S) lds[i] = v[k];
  }
  __syncthreads();
  for (int s = threadIdx.x; s < T.S; s += NT) grow[s] = lds[T.pre[s]];
}

// Ancestors-or-self path sums of the LDS vector x[] (preorder positions,
// x[ZERO] == 0), optionally weighted per position by wgt[] (global, padded
// with a 0 at ZERO is not required: the padding slot's x is 0): Euler-tour
// prefix scan.  Returns ps[] for own positions.  Reads x[] after the caller's
// barrier; writes `scan` (2*NT*CPT floats).  Two barriers.
template <int NT, int CPT, class Tables>
__device__ __forceinline__ void path_sum_euler(const Tables& O, const float* x, float* scan, float* wtot,
                                               float (&ps)[CPT], const float* wgt = nullptr) {
  constexpr int E = 2 * CPT;
  constexpr int NW = NT / 64;
  float ev[E];
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int p = O.ev[j] >> 1;
    const float xv = wgt ? x[p] * (p < O.ZERO ? wgt[p] : 0.0f) : x[p];
    ev[j] = (O.ev[j] & 1) ? -xv : xv;
  }
#pragma unroll
  for (int j = 1; j < E; ++j) ev[j] += ev[j - 1];
  const float tsum = ev[E - 1];
  const float ws = wave_scan_incl(tsum);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 63) wtot[w] = ws;
  __syncthreads();
  float off = ws - tsum;
#pragma unroll
  for (int i = 0; i < NW; ++i)
    if (i < w) off += wtot[i];
  float4* dst = reinterpret_cast<float4*>(scan + threadIdx.x * E);
#pragma unroll
  for (int j = 0; j < E; j += 4)
    dst[j / 4] = make_float4(ev[j] + off, ev[j + 1] + off, ev[j + 2] + off, ev[j + 3] + off);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < CPT; ++k) ps[k] = scan[O.tin[k]];
}

}  // namespace kb
