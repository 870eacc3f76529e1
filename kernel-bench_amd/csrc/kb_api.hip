// C-ABI of libkbench_hip: plan creation (device-resident layout tables built
// once per static problem) and the whole-pass drivers.  Declarations and the
// reference interface each entry point replaces are in include/kbench_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <climits>
#include <functional>
#include <map>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/kbench_hip.h"
#include "kb_kernels.hpp"

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace kb {
int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}
}  // namespace kb

namespace {

using kb::set_error;

#define KB_HIP(expr)                                                                       \
  do {                                                                                     \
    hipError_t _e = (expr);                                                                \
    if (_e != hipSuccess)                                                                  \
      return set_error(KB_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e));         \
  } while (0)

template <typename T>
int upload(T** dst, const std::vector<T>& src) {
  *dst = nullptr;
  if (src.empty()) return 0;
  KB_HIP(hipMalloc((void**)dst, src.size() * sizeof(T)));
  KB_HIP(hipMemcpy(*dst, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice));
  return 0;
}

template <typename T>
int alloc(T** dst, size_t n) {
  *dst = nullptr;
  if (n == 0) return 0;
  KB_HIP(hipMalloc((void**)dst, n * sizeof(T)));
  return 0;
}

}  // namespace

struct kb_plan {
  int S = 0, C = 0, n_fam = 0, n_waves = 0;
  int n_jump = 0, n_tlevels = 0, n_blevels = 0;
  std::vector<int> wave_start, wave_size, wave_split;
  // dependency levels: rows grouped by clade-DAG depth (0 = no splits); a row
  // only reads its own children, so level order is a valid schedule
  int n_levels = 0;
  std::vector<int> level_ptr;
  int* d_sched_rows = nullptr;
  // row classes: rows with identical inputs (same leaf, or same splits over
  // identical child classes) have identical forward outputs; the forward
  // computes one representative per class and copies it to the others, the
  // backward merges the adjoints of identical leaf rows (level 0)
  std::vector<int> f_level_ptr;        // representatives per level
  int* d_fsched = nullptr;             // representatives in level order
  int* d_fsplit_l = nullptr;           // split children remapped to representatives
  int* d_fsplit_r = nullptr;
  int n_copy = 0;                       // rows identical to an earlier representative
  int* d_dup_ptr = nullptr;             // [forward slots + 1] -> d_dup_rows
  int* d_dup_rows = nullptr;
  int n_cls0 = 0;                      // classes of level-0 rows
  int n_chunks0 = 0;                   // level-0 classes cut into chunks of <= KB_CHUNK0 members
  int* d_ck_ptr = nullptr;
  int* d_cls_ck_ptr = nullptr;
  unsigned char* b_ck_any = nullptr;
  int* d_rep_of = nullptr;             // [C] representative of each row
  int* d_m_side_ptr = nullptr;         // level-0 members (cls_rows order): staging sides
  int* d_m_side = nullptr;
  int* d_m_root = nullptr;
  float* d_dts = nullptr;              // [C, S] split terms stored by the forward (preorder rows)
  int64_t fwd_token = 0;               // counter of forwards on this plan
  const float* fwd_pi = nullptr;       // outputs of the forward with token fwd_token
  const float* fwd_pibar = nullptr;
  int* d_cls_ptr = nullptr;
  int* d_cls_rows = nullptr;
  int* d_row_kind = nullptr;  // 1: row of a leaf wave (leaf initialisation), 0: split row
  // device tables
  int* d_parent = nullptr; int* d_c1 = nullptr; int* d_c2 = nullptr; int* d_jump = nullptr;
  int* d_blevel_ptr = nullptr; int* d_blevel_node = nullptr;
  int* d_tlevel_ptr = nullptr; int* d_tlevel_node = nullptr;
  int* d_sub_start = nullptr; int* d_sub_end = nullptr;
  int* d_item = nullptr; int* d_leaf = nullptr; int* d_roots = nullptr;
  int* d_split_ptr = nullptr; int* d_split_l = nullptr; int* d_split_r = nullptr; float* d_split_lsp = nullptr;
  int* d_split_parent = nullptr;
  int* d_child_ptr = nullptr; int* d_child_in = nullptr;
  int* d_bslot = nullptr;  // [KB_BREC * C] the backward's record of every schedule slot
  float* d_unnorm = nullptr;
  // per-solve constants [S]
  float* c_DL = nullptr; float* c_SL1 = nullptr; float* c_SL2 = nullptr; float* c_pS = nullptr;
  float* c_pD = nullptr; float* c_colw = nullptr;
  float* lin_a = nullptr; float* lin_emc = nullptr; float* lin_k1 = nullptr; float* lin_k2 = nullptr;
  float* c_Ebar = nullptr; float* c_E = nullptr; float* c_mt = nullptr; float* c_col = nullptr;
  // preorder tables (see kb_rowops.hpp)
  int* d_pre = nullptr; int* d_pcol = nullptr; int* d_c1pos = nullptr; int* d_c2pos = nullptr; int* d_ppos = nullptr;
  int* d_pflag = nullptr; int* d_endpos = nullptr; int* d_tin = nullptr; int* d_euler = nullptr;
  int* d_post = nullptr;
  int* d_om_tab = nullptr;  // owner-major position tables of the large backward kernel (2048 < S <= 8192)
  int* d_euler_col = nullptr; int* d_tin_col = nullptr;  // the Euler tour in column terms
  kb::TreeScanDev tscan() const { return kb::TreeScanDev{S, d_pre, d_endpos, d_euler_col, d_tin_col}; }
  double* E64 = nullptr; int* n_e_iter = nullptr; double* loss_terms = nullptr; double* loss64 = nullptr;
  int* d_root_index = nullptr;
  int64_t n_splits = 0;
  // backward work (allocated on first use)
  float* b_staging = nullptr; unsigned char* b_split_on = nullptr; unsigned char* b_mask = nullptr;
  float* b_rhs0 = nullptr;
  float* b_rhsc = nullptr;
  unsigned char* b_m_mask = nullptr;
  unsigned char* b_cls_active = nullptr;
  float* b_contrib = nullptr; double* b_partial = nullptr; double* b_acc = nullptr; double* b_work = nullptr;
  float* b_om_const = nullptr;  // owner-major constants of the large backward kernel
  int* b_status = nullptr;
  int* h_status = nullptr;  // pinned host copy of b_status (kb_backward_stats)
  float* b_DL = nullptr; float* b_SL1 = nullptr; float* b_SL2 = nullptr; float* b_pS = nullptr; float* b_pD = nullptr;
  float* b_Ebar = nullptr; float* b_E = nullptr; float* b_mt = nullptr; float* b_col = nullptr;
  int b_nb_max = 0, b_n_partials = 0, b_variant = 0, b_large = 1;
  size_t b_slot = 0;  // floats per workgroup slot of b_contrib
  std::vector<int> b_poff;
  // kb_solve: rows of the families whose root lies at a level <= overlap_cut
  // come first in their level's backward schedule (n_early of them); those of
  // levels overlap_low .. overlap_cut are solved on a second stream while the
  // forward's later levels run, the levels below overlap_low as whole levels
  // afterwards
  int overlap_cut = -1;
  int overlap_low = 1;
  int overlap_grid = 1;  // workgroups of the early launches
  std::vector<int> n_early;
  hipStream_t s2 = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
  // optional per-launch timing of the wave kernels (HIP events on the launch stream)
  int prof = 0;
  std::vector<hipEvent_t> ev_fwd, ev_bwd;
  std::vector<void*> owned;

  kb::PreDev predev() const {
    kb::PreDev t;
    t.S = S;
    t.pre = d_pre;
    t.col = d_pcol;
    t.c1pos = d_c1pos;
    t.c2pos = d_c2pos;
    t.ppos = d_ppos;
    t.pflag = d_pflag;
    t.endpos = d_endpos;
    t.tin = d_tin;
    t.euler = d_euler;
    t.post = d_post;
    return t;
  }

  kb::TreeDev tree() const {
    kb::TreeDev t;
    t.S = S;
    t.n_jump = n_jump;
    t.n_blevels = n_blevels;
    t.parent = d_parent;
    t.c1 = d_c1;
    t.c2 = d_c2;
    t.jump = d_jump;
    t.blevel_ptr = d_blevel_ptr;
    t.blevel_node = d_blevel_node;
    t.sub_start = d_sub_start;
    t.sub_end = d_sub_end;
    return t;
  }
};

extern "C" {

const char* kb_last_error(void) { return g_last_error.c_str(); }

int kb_abi_version(void) { return KB_ABI_VERSION; }

void kb_plan_destroy(kb_plan* p) {
  if (!p) return;
  for (hipEvent_t e : p->ev_fwd) (void)hipEventDestroy(e);
  for (hipEvent_t e : p->ev_bwd) (void)hipEventDestroy(e);
  if (p->ev_fork) (void)hipEventDestroy(p->ev_fork);
  if (p->ev_join) (void)hipEventDestroy(p->ev_join);
  if (p->s2) (void)hipStreamDestroy(p->s2);
  for (void* ptr : p->owned)
    if (ptr) (void)hipFree(ptr);
  if (p->h_status) (void)hipHostFree(p->h_status);
  delete p;
}

int kb_plan_create(const kb_layout* L, kb_plan** out) {
  if (!L || !out) return set_error(KB_ERR_ARG, "null argument");
  *out = nullptr;
  const int S = L->S, C = L->C;
  if (S < 1 || C < 0) return set_error(KB_ERR_ARG, "bad sizes S=%d C=%d", S, C);
  if (S > 8192) return set_error(KB_ERR_ARG, "S=%d exceeds the supported maximum 8192", S);
  kb_plan* p = new kb_plan();
  p->S = S;
  p->C = C;
  p->n_fam = L->n_fam;
  p->n_waves = L->n_waves;

  // ---- species tree
  std::vector<int> parent(S), c1(S), c2(S), depth(S, -1), ss(S), se(S);
  for (int s = 0; s < S; ++s) {
    int64_t pa = L->node_parent[s];
    parent[s] = (pa >= 0 && pa < S) ? (int)pa : -1;
    int64_t a = L->node_child1[s], b = L->node_child2[s];
    c1[s] = (a >= 0 && a < S) ? (int)a : -1;
    c2[s] = (b >= 0 && b < S) ? (int)b : -1;
    ss[s] = (int)L->node_subtree_start[s];
    se[s] = (int)L->node_subtree_end[s];
  }
  // depth by walking to the root (bounded: a cycle is a layout error)
  int max_chain = 1;
  for (int s = 0; s < S; ++s) {
    int d = 0, cur = s;
    while (parent[cur] >= 0) {
      cur = parent[cur];
      if (++d > S) {
        kb_plan_destroy(p);
        return set_error(KB_ERR_ARG, "node_parent has a cycle");
      }
    }
    depth[s] = d;
    max_chain = std::max(max_chain, d + 1);
  }
  int n_jump = 0;
  while ((1 << n_jump) < max_chain) ++n_jump;
  std::vector<int> jump((size_t)std::max(n_jump, 1) * S, -1);
  for (int s = 0; s < S; ++s) jump[s] = parent[s];
  for (int t = 1; t < n_jump; ++t)
    for (int s = 0; s < S; ++s) {
      int a = jump[(size_t)(t - 1) * S + s];
      jump[(size_t)t * S + s] = a >= 0 ? jump[(size_t)(t - 1) * S + a] : -1;
    }
  int maxd = 0;
  for (int s = 0; s < S; ++s) maxd = std::max(maxd, depth[s]);
  std::vector<int> tptr(maxd + 2, 0), tnode;
  for (int d = 0; d <= maxd; ++d) {
    for (int s = 0; s < S; ++s)
      if (depth[s] == d) tnode.push_back(s);
    tptr[d + 1] = (int)tnode.size();
  }
  std::vector<int> bptr(1, 0), bnode;
  for (int d = maxd; d >= 0; --d) {
    bool any = false;
    for (int s = 0; s < S; ++s)
      if (depth[s] == d && (c1[s] >= 0 || c2[s] >= 0)) {
        bnode.push_back(s);
        any = true;
      }
    if (any) bptr.push_back((int)bnode.size());
  }
  // preorder (child1 first) and its Euler tour
  std::vector<int> pre(S, -1), pcol(S), c1pos(S), c2pos(S), ppos(S), pflag(S, 0), endpos(S), tin(S), euler;
  {
    int root = -1;
    for (int s = 0; s < S; ++s)
      if (parent[s] < 0) {
        if (root >= 0) {
          kb_plan_destroy(p);
          return set_error(KB_ERR_ARG, "node_parent has more than one root");
        }
        root = s;
      }
    if (root < 0) {
      kb_plan_destroy(p);
      return set_error(KB_ERR_ARG, "node_parent has no root");
    }
    std::vector<int> stack{root};
    int order = 0;
    while (!stack.empty()) {
      int v = stack.back();
      stack.pop_back();
      pre[v] = order;
      pcol[order] = v;
      ++order;
      if (c2[v] >= 0) stack.push_back(c2[v]);
      if (c1[v] >= 0) stack.push_back(c1[v]);
    }
    if (order != S) {
      kb_plan_destroy(p);
      return set_error(KB_ERR_ARG, "species tree is not connected (%d of %d nodes reachable)", order, S);
    }
    std::vector<int> size(S, 1);
    for (int i = S - 1; i >= 0; --i) {
      int v = pcol[i];
      if (c1[v] >= 0) size[v] += size[c1[v]];
      if (c2[v] >= 0) size[v] += size[c2[v]];
    }
    for (int i = 0; i < S; ++i) {
      int v = pcol[i];
      c1pos[i] = c1[v] >= 0 ? pre[c1[v]] : -1;
      c2pos[i] = c2[v] >= 0 ? pre[c2[v]] : -1;
      ppos[i] = parent[v] >= 0 ? pre[parent[v]] : -1;
      pflag[i] = (parent[v] >= 0 && c1[parent[v]] == v) ? 1 : 0;
      endpos[i] = i + size[v];
    }
    std::vector<int> open;
    for (int i = 0; i < S; ++i) {
      while (!open.empty() && endpos[open.back()] <= i) {
        euler.push_back((open.back() << 1) | 1);
        open.pop_back();
      }
      tin[i] = (int)euler.size();
      euler.push_back(i << 1);
      open.push_back(i);
    }
    while (!open.empty()) {
      euler.push_back((open.back() << 1) | 1);
      open.pop_back();
    }
  }
  p->n_jump = n_jump;
  p->n_tlevels = maxd + 1;
  p->n_blevels = (int)bptr.size() - 1;

  // ---- rows, splits, waves (int64 values range-checked before narrowing)
  std::vector<int> item(C), leaf(C), roots(L->n_fam);
  for (int r = 0; r < C; ++r) {
    const int64_t it = L->rate_item_idx[r], lf = L->leaf_state_index[r];
    if (it != 0) {  // one parameter row: the whole-pass kernels address every constant at row 0
      kb_plan_destroy(p);
      return set_error(KB_ERR_ARG, "rate_item_idx[%d]=%lld: the whole-pass driver needs every row in item 0", r,
                       (long long)it);
    }
    if (lf < -1 || lf >= S) {
      kb_plan_destroy(p);
      return set_error(KB_ERR_ARG, "leaf_state_index[%d]=%lld: leaf state outside [-1,%d)", r, (long long)lf, S);
    }
    item[r] = 0;
    leaf[r] = (int)lf;
  }
  for (int f = 0; f < L->n_fam; ++f) {
    const int64_t rt = L->root_row_ids[f];
    if (rt < 0 || rt >= C) {
      kb_plan_destroy(p);
      return set_error(KB_ERR_ARG, "root_row_ids[%d]=%lld outside [0,%d)", f, (long long)rt, C);
    }
    roots[f] = (int)rt;
  }
  const int64_t NS = L->n_splits;
  if (NS < 0 || NS >= (int64_t{1} << 29)) {  // split sides are ints below 2^30
    kb_plan_destroy(p);
    return set_error(KB_ERR_ARG, "n_splits %lld outside [0, 2^29)", (long long)NS);
  }
  // rows -> wave; every wave a contiguous row range, in order
  std::vector<int> wave_of(C, -1);
  for (int w = 0; w < L->n_waves; ++w) {
    const int64_t b = L->wave_start[w], e = b + L->wave_size[w];
    if (b < 0 || e > C || L->wave_size[w] < 0) {
      kb_plan_destroy(p);
      return set_error(KB_ERR_ARG, "wave %d covers rows [%lld,%lld) outside [0,%d)", w, (long long)b, (long long)e, C);
    }
    for (int64_t r = b; r < e; ++r) {
      if (wave_of[r] >= 0) {
        kb_plan_destroy(p);
        return set_error(KB_ERR_ARG, "row %lld lies in waves %d and %d", (long long)r, wave_of[r], w);
      }
      wave_of[r] = w;
    }
  }
  for (int r = 0; r < C; ++r)
    if (wave_of[r] < 0) {
      kb_plan_destroy(p);
      return set_error(KB_ERR_ARG, "row %d lies in no wave", r);
    }
  std::vector<int> cnt(C + 1, 0);
  for (int64_t i = 0; i < NS; ++i) {
    int64_t pr = L->split_parent[i];
    if (pr < 0 || pr >= C) {
      kb_plan_destroy(p);
      return set_error(KB_ERR_ARG, "split %lld has parent row %lld outside [0,%d)", (long long)i, (long long)pr, C);
    }
    int64_t a = L->split_left[i], b = L->split_right[i];
    if (a < 0 || a >= C || b < 0 || b >= C || wave_of[pr] < 0 || wave_of[a] < 0 || wave_of[b] < 0 ||
        wave_of[a] >= wave_of[pr] || wave_of[b] >= wave_of[pr]) {
      kb_plan_destroy(p);
      return set_error(KB_ERR_ARG, "split %lld children (%lld,%lld) must lie in waves before parent row %lld",
                       (long long)i, (long long)a, (long long)b, (long long)pr);
    }
    cnt[pr + 1]++;
  }
  for (int r = 0; r < C; ++r) cnt[r + 1] += cnt[r];
  std::vector<int> sptr(cnt), fill(cnt.begin(), cnt.end() - 1);
  std::vector<int> sl(NS), sr(NS), spar(NS);
  std::vector<float> slsp(NS);
  for (int64_t i = 0; i < NS; ++i) {  // stable: keeps the layout's split order per parent
    int pr = (int)L->split_parent[i];
    int pos = fill[pr]++;
    sl[pos] = (int)L->split_left[i];
    sr[pos] = (int)L->split_right[i];
    slsp[pos] = (float)L->split_log_prob[i];
    spar[pos] = pr;
  }
  // child -> incoming (split, side) CSR in increasing split order: fixed gather order
  std::vector<int> ccnt(C + 1, 0);
  for (int64_t i = 0; i < NS; ++i) {
    ccnt[sl[i] + 1]++;
    ccnt[sr[i] + 1]++;
  }
  for (int r = 0; r < C; ++r) ccnt[r + 1] += ccnt[r];
  std::vector<int> cfill(ccnt.begin(), ccnt.end() - 1), cin(2 * NS);
  for (int64_t i = 0; i < NS; ++i) {
    cin[cfill[sl[i]]++] = (int)(2 * i);
    cin[cfill[sr[i]]++] = (int)(2 * i + 1);
  }
  for (int w = 0; w < L->n_waves; ++w) {
    p->wave_start.push_back((int)L->wave_start[w]);
    p->wave_size.push_back((int)L->wave_size[w]);
    p->wave_split.push_back(L->wave_has_splits[w] ? 1 : 0);
  }
  std::vector<float> unnorm(L->unnorm_row_max, L->unnorm_row_max + S);
  std::vector<int> root_index(C, -1);
  for (int f = 0; f < L->n_fam; ++f) root_index[roots[f]] = f;
  p->n_splits = NS;
  // DAG depth of every row (children precede parents: checked above)
  std::vector<int> row_kind(C, 0), dagd(C, 0);
  for (int w = 0; w < L->n_waves; ++w)
    for (int64_t r = L->wave_start[w]; r < L->wave_start[w] + L->wave_size[w]; ++r)
      row_kind[r] = L->wave_has_splits[w] ? 0 : 1;
  for (int r = 0; r < C; ++r)
    if (row_kind[r] && (leaf[r] < 0 || leaf[r] >= S)) {  // the leaf term indexes the state
      kb_plan_destroy(p);
      return set_error(KB_ERR_ARG, "leaf row %d has leaf state %d outside [0,%d)", r, leaf[r], S);
    }
  for (int r = 0; r < C; ++r)
    for (int i = sptr[r]; i < sptr[r + 1]; ++i) dagd[r] = std::max(dagd[r], 1 + std::max(dagd[sl[i]], dagd[sr[i]]));
  int maxdag = 0;
  for (int r = 0; r < C; ++r) maxdag = std::max(maxdag, dagd[r]);
  p->n_levels = C > 0 ? maxdag + 1 : 0;
  p->level_ptr.assign(p->n_levels + 1, 0);
  for (int r = 0; r < C; ++r) p->level_ptr[dagd[r] + 1]++;
  for (int d = 0; d < p->n_levels; ++d) p->level_ptr[d + 1] += p->level_ptr[d];
  std::vector<int> sched(C), lfill(p->level_ptr.begin(), p->level_ptr.end() - 1);
  for (int r = 0; r < C; ++r) sched[lfill[dagd[r]]++] = r;

  // ---- row classes (hash-consing in dependency order; KB_DEDUP=0 disables)
  std::vector<int> cls(C, -1), rep;
  {
    const char* env = getenv("KB_DEDUP");
    const bool dedup = !(env && env[0] == '0');
    std::map<std::vector<int64_t>, int> ids;
    std::vector<std::array<int64_t, 3>> trip;
    for (int r : sched) {  // children precede parents
      std::vector<int64_t> key;
      if (!dedup) {
        key = {2, r};
      } else if (row_kind[r] || sptr[r] == sptr[r + 1]) {
        key = {row_kind[r] ? 0 : 3, leaf[r], item[r], row_kind[r] ? 0 : r};
      } else {
        trip.clear();
        for (int i = sptr[r]; i < sptr[r + 1]; ++i) {
          int64_t a = cls[sl[i]], b = cls[sr[i]];
          int64_t bits;
          std::memcpy(&bits, &slsp[i], sizeof(bits));
          trip.push_back({std::min(a, b), std::max(a, b), bits});
        }
        std::sort(trip.begin(), trip.end());
        key = {1, item[r]};
        for (auto& t3 : trip) key.insert(key.end(), t3.begin(), t3.end());
      }
      auto it = ids.find(key);
      if (it == ids.end()) {
        it = ids.emplace(std::move(key), (int)rep.size()).first;
        rep.push_back(r);
      }
      cls[r] = it->second;
    }
  }
  std::vector<int> fsched, fsl(NS), fsr(NS), copy_dst, copy_src;
  p->f_level_ptr.assign(p->n_levels + 1, 0);
  for (int r : sched)
    if (rep[cls[r]] == r) {
      fsched.push_back(r);
      p->f_level_ptr[dagd[r] + 1]++;
    } else {
      copy_dst.push_back(r);
      copy_src.push_back(rep[cls[r]]);
    }
  for (int d = 0; d < p->n_levels; ++d) p->f_level_ptr[d + 1] += p->f_level_ptr[d];
  for (int64_t i = 0; i < NS; ++i) {
    fsl[i] = rep[cls[sl[i]]];
    fsr[i] = rep[cls[sr[i]]];
  }
  p->n_copy = (int)copy_dst.size();
  // level-0 classes for the backward (members in increasing row order, representative first)
  std::vector<int> cls_ptr{0}, cls_rows;
  {
    std::map<int, std::vector<int>> members;
    for (int k = 0; k < (C > 0 ? p->level_ptr[1] : 0); ++k) members[cls[sched[k]]].push_back(sched[k]);
    std::vector<std::vector<int>*> order;
    for (auto& kv : members) order.push_back(&kv.second);
    std::sort(order.begin(), order.end(), [](auto* x, auto* y) { return (*x)[0] < (*y)[0]; });
    for (auto* m : order) {
      std::sort(m->begin(), m->end());
      cls_rows.insert(cls_rows.end(), m->begin(), m->end());
      cls_ptr.push_back((int)cls_rows.size());
    }
  }
  p->n_cls0 = (int)cls_ptr.size() - 1;
  // chunks of at most KB_CHUNK0 members of a level-0 class (nearly equal sizes)
  std::vector<int> ck_ptr{0}, cls_ck_ptr{0};
  for (int c = 0; c < p->n_cls0; ++c) {
    const int b = cls_ptr[c], n = cls_ptr[c + 1] - b;
    const int pieces = (n + kb::KB_CHUNK0 - 1) / kb::KB_CHUNK0;
    for (int k = 1; k <= pieces; ++k) ck_ptr.push_back(b + (int)((int64_t)n * k / pieces));
    cls_ck_ptr.push_back((int)ck_ptr.size() - 1);
  }
  p->n_chunks0 = (int)ck_ptr.size() - 1;

  int rc = 0;
  rc |= upload(&p->d_parent, parent);
  rc |= upload(&p->d_c1, c1);
  rc |= upload(&p->d_c2, c2);
  rc |= upload(&p->d_jump, jump);
  rc |= upload(&p->d_blevel_ptr, bptr);
  rc |= upload(&p->d_blevel_node, bnode);
  rc |= upload(&p->d_tlevel_ptr, tptr);
  rc |= upload(&p->d_tlevel_node, tnode);
  rc |= upload(&p->d_sub_start, ss);
  rc |= upload(&p->d_sub_end, se);
  rc |= upload(&p->d_item, item);
  rc |= upload(&p->d_leaf, leaf);
  rc |= upload(&p->d_roots, roots);
  rc |= upload(&p->d_split_ptr, sptr);
  rc |= upload(&p->d_split_l, sl);
  rc |= upload(&p->d_split_r, sr);
  rc |= upload(&p->d_split_lsp, slsp);
  rc |= upload(&p->d_split_parent, spar);
  rc |= upload(&p->d_child_ptr, ccnt);
  rc |= upload(&p->d_child_in, cin);
  rc |= upload(&p->d_unnorm, unnorm);
  rc |= upload(&p->d_root_index, root_index);
  {
    // kb_solve's overlap (KB_OVERLAP_CUT = c): every row of a family whose
    // root lies at level <= c moves to the front of its level's backward
    // schedule, in row order, the other rows after it, also in row order
    // (kb_backward runs each level's rows in this order too, in one launch).
    // An early row must have early parents only, and its children must be
    // early as well: families that share a row are grouped (union-find) and a
    // group is early when all of its roots are; rows no root reaches stay late.
    std::vector<int> fam_of(C, -1), grp(L->n_fam);
    for (int f = 0; f < L->n_fam; ++f) grp[f] = f;
    std::function<int(int)> find = [&](int f) { return grp[f] == f ? f : (grp[f] = find(grp[f])); };
    for (int f = 0; f < L->n_fam; ++f) {
      std::vector<int> stack{roots[f]};
      while (!stack.empty()) {
        const int r = stack.back();
        stack.pop_back();
        if (fam_of[r] >= 0) {
          const int a = find(fam_of[r]), b = find(f);
          if (a != b) grp[a] = b;
          continue;
        }
        fam_of[r] = f;
        for (int i = sptr[r]; i < sptr[r + 1]; ++i) {
          stack.push_back(sl[i]);
          stack.push_back(sr[i]);
        }
      }
    }
    std::vector<int> grp_top(L->n_fam, 0);
    for (int f = 0; f < L->n_fam; ++f) grp_top[find(f)] = std::max(grp_top[find(f)], dagd[roots[f]]);
    std::vector<int> row_top(C, INT_MAX);
    for (int r = 0; r < C; ++r)
      if (fam_of[r] >= 0) row_top[r] = grp_top[find(fam_of[r])];
    // The early launches get KB_OVERLAP_GRID workgroups (default 5/8 of the
    // CUs, one backward workgroup per CU); the cut defaults to the highest level
    // whose forward rows would not fit on the other CUs (two forward workgroups
    // per CU, one for rows past 4096 states), so the forward's later levels run
    // beside the early rows without waiting for CUs; with fewer early rows than
    // CUs in the early launches there is nothing worth overlapping and the cut
    // is -1.
    int dev = 0, n_cu = 1;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n_cu = 1;
    const char* gv = getenv("KB_OVERLAP_GRID");
    p->overlap_grid = std::max(1, gv && atoi(gv) > 0 ? atoi(gv) : n_cu * 5 / 8);
    const char* cv = getenv("KB_OVERLAP_CUT");
    int cut = -1;
    if (cv) {
      cut = atoi(cv);
    } else if (p->n_levels >= 3) {
      const int cap = std::max(1, n_cu - p->overlap_grid) * (S > 4096 ? 1 : 2);
      cut = p->n_levels - 1;
      while (cut >= 1 && p->f_level_ptr[cut + 1] - p->f_level_ptr[cut] <= cap) --cut;
    }
    if (cut >= p->n_levels - 1) cut = p->n_levels - 2;
    p->n_early.assign(std::max(p->n_levels, 1), 0);
    for (int d = 1; d < p->n_levels; ++d) {
      const int b = p->level_ptr[d], e = p->level_ptr[d + 1];
      std::stable_partition(sched.begin() + b, sched.begin() + e, [&](int r) { return row_top[r] <= cut; });
      int ne = 0;
      for (int k = b; k < e; ++k) ne += row_top[sched[k]] <= cut ? 1 : 0;
      p->n_early[d] = ne;
    }
    // The early launches run the cut's levels down to overlap_low; below it
    // the levels run whole, on every CU, after both streams have met.  The
    // default low is the lowest level at which the early launches (their rows
    // in rounds of one row per workgroup) still take no longer than what runs
    // on the other CUs meanwhile: the forward's later levels (a round there
    // counted as 0.8 of a backward round) and the late rows of the levels
    // down to low.  With more early rows the early stream would hold 5/8 of
    // the CUs for most of the backward.  A cut given by KB_OVERLAP_CUT keeps
    // low = 1 unless KB_OVERLAP_LOW says otherwise.
    const char* lv = getenv("KB_OVERLAP_LOW");
    int low = 1;
    if (lv) {
      low = std::max(1, atoi(lv));
    } else if (cut >= 1 && !cv) {
      const int g = std::max(1, p->overlap_grid), rest = std::max(1, n_cu - g);
      const int kf = S > 4096 ? 1 : 2;
      double mf = 0.0;
      for (int d = cut + 1; d < p->n_levels; ++d) {
        const int nf = p->f_level_ptr[d + 1] - p->f_level_ptr[d];
        mf += 0.8 * ((nf + kf * rest - 1) / (kf * rest));
      }
      auto rounds = [](long n, long w) { return (double)((n + w - 1) / w); };
      for (low = 1; low <= cut; ++low) {
        double e = 0.0, ml = 0.0;
        for (int d = low; d <= cut; ++d) e += rounds(p->n_early[d], g);
        for (int d = low; d < p->n_levels; ++d)
          ml += rounds(p->level_ptr[d + 1] - p->level_ptr[d] - (d <= cut ? p->n_early[d] : 0), rest);
        if (e <= mf + ml) break;
      }
      int ne = 0;
      for (int d = low; d <= cut; ++d) ne += p->n_early[d];
      if (ne < n_cu) low = cut + 1;
    }
    p->overlap_low = low;
    if (low > cut) cut = -1;
    p->overlap_cut = cut;
  }
  rc |= upload(&p->d_sched_rows, sched);
  rc |= upload(&p->d_fsched, fsched);
  rc |= upload(&p->d_fsplit_l, fsl);
  rc |= upload(&p->d_fsplit_r, fsr);
  {
    // per forward slot (representative), its identical rows
    std::vector<int> slot_of(C, -1);
    for (size_t j = 0; j < fsched.size(); ++j) slot_of[fsched[j]] = (int)j;
    std::vector<int> dptr(fsched.size() + 1, 0), drows(copy_dst.size());
    for (size_t k = 0; k < copy_dst.size(); ++k) dptr[slot_of[copy_src[k]] + 1]++;
    for (size_t j = 0; j < fsched.size(); ++j) dptr[j + 1] += dptr[j];
    std::vector<int> dfill(dptr.begin(), dptr.end() - 1);
    for (size_t k = 0; k < copy_dst.size(); ++k) drows[dfill[slot_of[copy_src[k]]]++] = copy_dst[k];
    rc |= upload(&p->d_dup_ptr, dptr);
    rc |= upload(&p->d_dup_rows, drows);
  }
  rc |= upload(&p->d_cls_ptr, cls_ptr);
  rc |= upload(&p->d_ck_ptr, ck_ptr);
  rc |= upload(&p->d_cls_ck_ptr, cls_ck_ptr);
  rc |= upload(&p->d_cls_rows, cls_rows);
  {
    std::vector<int> rep_of(C);
    for (int r = 0; r < C; ++r) rep_of[r] = rep[cls[r]];
    rc |= upload(&p->d_rep_of, rep_of);
    // the backward's record of schedule slot j (row sched[j]), KB_BREC ints
    std::vector<int> brec((size_t)kb::KB_BREC * C, -1);
    for (int j = 0; j < C; ++j) {
      const int r = sched[j], gb = ccnt[r], n = ccnt[r + 1] - gb;
      int* q = brec.data() + (size_t)kb::KB_BREC * j;
      q[kb::BR_S0] = n > 0 ? cin[gb] : -1;
      q[kb::BR_S1] = n > 1 ? (cin[gb + 1] | (n > 2 ? (1 << 30) : 0)) : -1;
      q[kb::BR_ROW] = r;
      q[kb::BR_FAM] = root_index[r];
      q[kb::BR_LEAF] = row_kind[r];
      q[kb::BR_SB] = sptr[r];
      q[kb::BR_SE] = sptr[r + 1];
      q[kb::BR_REP] = rep_of[r];
      const bool hs = sptr[r + 1] > sptr[r];
      q[kb::BR_L0] = hs ? sl[sptr[r]] : -1;
      q[kb::BR_R0] = hs ? sr[sptr[r]] : -1;
      int lsp_bits = 0;
      if (hs) std::memcpy(&lsp_bits, &slsp[sptr[r]], sizeof(lsp_bits));
      q[kb::BR_LSP0] = lsp_bits;
      q[kb::BR_LPOS] = row_kind[r] ? pre[leaf[r]] : -1;
    }
    rc |= upload(&p->d_bslot, brec);
    std::vector<int> msp{0}, ms, mroot;
    for (int r : cls_rows) {
      for (int j = ccnt[r]; j < ccnt[r + 1]; ++j) ms.push_back(cin[j]);
      msp.push_back((int)ms.size());
      mroot.push_back(root_index[r]);
    }
    rc |= upload(&p->d_m_side_ptr, msp);
    rc |= upload(&p->d_m_side, ms);
    rc |= upload(&p->d_m_root, mroot);
  }
  rc |= alloc(&p->d_dts, (size_t)std::max(1, C) * S);
  rc |= upload(&p->d_pre, pre);
  rc |= upload(&p->d_pcol, pcol);
  rc |= upload(&p->d_c1pos, c1pos);
  rc |= upload(&p->d_c2pos, c2pos);
  rc |= upload(&p->d_ppos, ppos);
  rc |= upload(&p->d_pflag, pflag);
  rc |= upload(&p->d_endpos, endpos);
  rc |= upload(&p->d_tin, tin);
  rc |= upload(&p->d_euler, euler);
  {
    std::vector<int> post;
    post.reserve(S);
    for (int e : euler)
      if (e & 1) post.push_back(e >> 1);
    rc |= upload(&p->d_post, post);
    if (S > 1024 && S <= 8192) {
      // owner-major position tables of bwd_row_large_kernel (kb::OmTab)
      const int ld = kb::kb_large_ld(S), nt = kb::kb_large_nt(S), cpt = ld / nt, zero = ld;
      std::vector<int> om((size_t)kb::KB_OM_TABS * ld);
      for (int i = 0; i < ld; ++i) {
        const size_t o = (size_t)(i % cpt) * nt + i / cpt;
        const bool ok = i < S;
        om[kb::OMT_C1 * (size_t)ld + o] = ok ? c1pos[i] : -1;
        om[kb::OMT_C2 * (size_t)ld + o] = ok ? c2pos[i] : -1;
        const int pa = ok && ppos[i] >= 0 ? ppos[i] : zero;
        const int e1 = ok ? endpos[i] - 1 : zero;
        om[kb::OMT_PK * (size_t)ld + o] = pa | (e1 << 16) | ((ok && ppos[i] >= 0 && pflag[i]) ? (1 << 30) : 0);
        om[kb::OMT_PN * (size_t)ld + o] = ok ? (post[i] | ((tin[i] - i) << 16)) : zero;
      }
      rc |= upload(&p->d_om_tab, om);
    }
  }
  {
    std::vector<int> ecol(euler.size()), tcol(S);
    for (size_t q = 0; q < euler.size(); ++q) ecol[q] = (pcol[euler[q] >> 1] << 1) | (euler[q] & 1);
    for (int s = 0; s < S; ++s) tcol[s] = tin[pre[s]];
    rc |= upload(&p->d_euler_col, ecol);
    rc |= upload(&p->d_tin_col, tcol);
  }
  rc |= alloc(&p->c_Ebar, S);
  rc |= alloc(&p->c_E, S);
  rc |= alloc(&p->c_mt, S);
  rc |= alloc(&p->c_col, S);
  rc |= upload(&p->d_row_kind, row_kind);
  rc |= alloc(&p->c_DL, S);
  rc |= alloc(&p->c_SL1, S);
  rc |= alloc(&p->c_SL2, S);
  rc |= alloc(&p->c_pS, S);
  rc |= alloc(&p->c_pD, S);
  rc |= alloc(&p->c_colw, S);
  rc |= alloc(&p->lin_a, S);
  rc |= alloc(&p->lin_emc, S);
  rc |= alloc(&p->lin_k1, S);
  rc |= alloc(&p->lin_k2, S);
  rc |= alloc(&p->E64, S);
  rc |= alloc(&p->n_e_iter, 1);
  rc |= alloc(&p->loss_terms, std::max(1, L->n_fam));
  rc |= alloc(&p->loss64, 1);
  for (void* ptr : {(void*)p->d_parent, (void*)p->d_c1, (void*)p->d_c2, (void*)p->d_jump, (void*)p->d_blevel_ptr,
                    (void*)p->d_blevel_node, (void*)p->d_tlevel_ptr, (void*)p->d_tlevel_node, (void*)p->d_sub_start,
                    (void*)p->d_sub_end, (void*)p->d_item, (void*)p->d_leaf, (void*)p->d_roots, (void*)p->d_split_ptr,
                    (void*)p->d_split_l, (void*)p->d_split_r, (void*)p->d_split_lsp, (void*)p->d_split_parent,
                    (void*)p->d_child_ptr, (void*)p->d_child_in, (void*)p->d_bslot, (void*)p->d_unnorm, (void*)p->c_DL, (void*)p->c_SL1,
                    (void*)p->c_SL2, (void*)p->c_pS, (void*)p->c_pD, (void*)p->c_colw, (void*)p->lin_a,
                    (void*)p->lin_emc, (void*)p->lin_k1, (void*)p->lin_k2, (void*)p->E64, (void*)p->n_e_iter,
                    (void*)p->loss_terms, (void*)p->loss64, (void*)p->d_root_index,
                    (void*)p->d_sched_rows, (void*)p->d_row_kind, (void*)p->d_pre, (void*)p->d_pcol,
                    (void*)p->d_fsched, (void*)p->d_fsplit_l, (void*)p->d_fsplit_r, (void*)p->d_dup_ptr,
                    (void*)p->d_dup_rows, (void*)p->d_cls_ptr, (void*)p->d_cls_rows, (void*)p->d_ck_ptr, (void*)p->d_cls_ck_ptr, (void*)p->d_rep_of, (void*)p->d_m_side_ptr, (void*)p->d_m_side, (void*)p->d_m_root,
                    (void*)p->d_dts,
                    (void*)p->d_c1pos, (void*)p->d_c2pos, (void*)p->d_ppos, (void*)p->d_pflag, (void*)p->d_endpos,
                    (void*)p->d_tin, (void*)p->d_euler, (void*)p->d_post, (void*)p->d_om_tab, (void*)p->d_euler_col, (void*)p->d_tin_col, (void*)p->c_Ebar, (void*)p->c_E, (void*)p->c_mt,
                    (void*)p->c_col})
    p->owned.push_back(ptr);
  if (rc) {
    kb_plan_destroy(p);
    return KB_ERR_HIP;
  }
  *out = p;
  return 0;
}

int kb_plan_info(const kb_plan* p, int32_t* out, int n) {
  if (!p || !out) return set_error(KB_ERR_ARG, "null argument");
  const int32_t n_fwd = p->f_level_ptr.empty() ? 0 : p->f_level_ptr.back();
  const int32_t rows0 = p->level_ptr.size() > 1 ? p->level_ptr[1] : 0;
  int32_t n_early = 0;
  for (int d = p->overlap_low; d <= p->overlap_cut; ++d) n_early += p->n_early[d];
  int32_t v[13] = {p->S,      p->C,      p->n_fam,  p->n_waves,       p->n_jump,       p->n_blevels, p->n_levels,
                   n_fwd,     p->n_cls0, rows0,     p->overlap_cut, n_early, p->overlap_low};
  for (int i = 0; i < n && i < 13; ++i) out[i] = v[i];
  return 0;
}

}  // extern "C"

// The forward in three parts (kb_forward runs them in order; kb_solve
// interleaves the backward's early rows with the levels): checks, E-step and
// the row kernels' parameters; one dependency level; the loss.
static int forward_setup(kb_plan* p, const kb_forward_io* io, hipStream_t st, kb::FwdParams& F) {
  if (!p || !io) return set_error(KB_ERR_ARG, "null argument");
  if (io->pi_iters < 2 || io->pi_iters % 2 != 0)
    return set_error(KB_ERR_ARG, "pi_iters must be an even integer at least 2");
  if (io->e_max_iter < 1) return set_error(KB_ERR_ARG, "e_max_iter must be at least 1");
  if (!(io->e_tol > 0.0)) return set_error(KB_ERR_ARG, "e_tol must be positive");
  const int S = p->S;

  kb::EStepParams E{};
  E.tr = p->tree();
  E.ts = p->tscan();
  E.pd = p->predev();
  E.S = S;
  E.n_tlevels = p->n_tlevels;
  E.tlevel_ptr = p->d_tlevel_ptr;
  E.tlevel_node = p->d_tlevel_node;
  E.theta = io->theta;
  E.statewise = io->statewise;
  E.col_weights = io->col_weights;
  E.use_col = io->use_col_weights;
  E.unnorm_row_max = p->d_unnorm;
  E.e_init = io->e_init;
  E.max_iter = io->e_max_iter;
  E.tol = io->e_tol;
  E.E = io->E;
  E.E_s1 = io->E_s1;
  E.E_s2 = io->E_s2;
  E.Ebar = io->Ebar;
  E.log_pS = io->log_pS;
  E.log_pD = io->log_pD;
  E.log_pL = io->log_pL;
  E.mt = io->max_coupling;
  E.col_log_probs = io->col_log_probs;
  E.E64 = p->E64;
  E.n_iter_out = p->n_e_iter;
  E.c_DL = p->c_DL;
  E.c_SL1 = p->c_SL1;
  E.c_SL2 = p->c_SL2;
  E.c_pS = p->c_pS;
  E.c_pD = p->c_pD;
  E.c_colw = p->c_colw;
  E.c_Ebar = p->c_Ebar;
  E.c_E = p->c_E;
  E.c_mt = p->c_mt;
  E.c_col = p->c_col;
  E.pre = p->d_pre;
  E.lin_a = p->lin_a;
  E.lin_emc = p->lin_emc;
  E.lin_k1 = p->lin_k1;
  E.lin_k2 = p->lin_k2;
  kb::launch_estep(E, st);
  KB_HIP(hipGetLastError());

  F = kb::FwdParams{};
  F.tr = p->tree();
  F.S = S;
  F.n_sweeps = io->pi_iters - 1;
  F.use_col = io->use_col_weights;
  F.lin_a = p->lin_a;
  F.lin_emc = p->lin_emc;
  F.lin_k1 = p->lin_k1;
  F.lin_k2 = p->lin_k2;
  F.pre = p->predev();
  {
    // KB_FWD_WIDE: 1 = 256 x 8, 2 = 1024 x 2 on every level, 3 = the size-based
    // shapes without the narrow one (tuning / test knob); default 0
    const char* w = getenv("KB_FWD_WIDE");
    F.wide = (w && (w[0] == '1' || w[0] == '2' || w[0] == '3')) ? w[0] - '0' : 0;
    // 512 x 4 keeps three rows per CU resident, 1024 x 2 two rows with a
    // shorter per-row latency.  Measured per level on rows of 1025..2048
    // states (config 3): the narrow shape wins on levels of less than one row
    // per CU and on the leaf level (no split term; the last round of 512 x 4
    // rows would run one row per CU), the 512 x 4 shape on the others (levels
    // of 570..1428 rows: 4-6 us each).  Shorter rows keep the earlier rule,
    // the narrow shape below six rows per CU.
    int dev = 0, n_cu = 0;
    KB_HIP(hipGetDevice(&dev));
    KB_HIP(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
    F.narrow_below = S > 1024 ? n_cu : 6 * n_cu;
  }
  F.colw = p->c_colw;
  F.col = p->c_col;
  F.mt = p->c_mt;
  F.DL = p->c_DL;
  F.Ebar = p->c_Ebar;
  F.E = p->c_E;
  F.SL1 = p->c_SL1;
  F.SL2 = p->c_SL2;
  F.pD = p->c_pD;
  F.pS = p->c_pS;
  F.leaf_state = p->d_leaf;
  F.split_ptr = p->d_split_ptr;
  F.split_l = p->d_fsplit_l;
  F.split_r = p->d_fsplit_r;
  F.split_lsp = p->d_split_lsp;
  F.pi = io->pi;
  F.pibar = io->pibar;
  F.rowmax = io->pibar_row_max;
  F.sched_rows = p->d_fsched;
  F.row_kind = p->d_row_kind;
  F.dup_ptr = p->d_dup_ptr;
  F.dup_rows = p->d_dup_rows;
  F.om_tab = p->d_om_tab;
  {
    // rows of 4097..8192 states: the contiguous-ownership kernel on the
    // owner-major tables (KB_FWD_LARGE=0: the Euler-tour kernel)
    const char* lv = getenv("KB_FWD_LARGE");
    F.large = (lv && lv[0] == '0') ? 0 : 1;
  }
  F.dts_out = p->d_dts;
  p->fwd_token += 1;
  p->fwd_pi = io->pi;
  p->fwd_pibar = io->pibar;
  return 0;
}

static int forward_level(kb_plan* p, kb::FwdParams& F, int d, hipStream_t st) {
  if (p->prof) KB_HIP(hipEventRecord(p->ev_fwd[2 * d], st));
  const int nb = F.narrow_below;
  if (d == 0 && p->S > 1024) F.narrow_below = INT_MAX;  // the leaf level
  kb::launch_fwd_wave(F, p->f_level_ptr[d], p->f_level_ptr[d + 1] - p->f_level_ptr[d], st);
  F.narrow_below = nb;
  if (p->prof) KB_HIP(hipEventRecord(p->ev_fwd[2 * d + 1], st));
  return 0;
}

static int forward_finish(kb_plan* p, const kb_forward_io* io, hipStream_t st) {
  KB_HIP(hipGetLastError());
  kb::launch_loss(io->pi, p->d_roots, io->E, p->S, p->n_fam, p->loss_terms, p->loss64, io->loss, st);
  KB_HIP(hipGetLastError());
  return 0;
}

extern "C" int kb_forward(kb_plan* p, const kb_forward_io* io, void* stream) {
  hipStream_t st = (hipStream_t)stream;
  kb::FwdParams F{};
  int rc = forward_setup(p, io, st, F);
  for (int d = 0; !rc && d < p->n_levels; ++d) rc = forward_level(p, F, d, st);
  return rc ? rc : forward_finish(p, io, st);
}

// floats per workgroup slot of the backward row kernels
static size_t bwd_slot_floats(int S, int large) {
  return kb::kb_use_large(S, large) ? (size_t)kb::KB_LARGE_SLOT_ROWS * kb::kb_large_ld(S)
                                    : (size_t)8 * kb::kb_slot_ld(S, large);
}

static int ensure_backward_work(kb_plan* p, int use_col) {
  const int S = p->S, C = p->C;
  // resident workgroups of the backward row kernel: its per-level grid
  int dev = 0, n_cu = 0;
  KB_HIP(hipGetDevice(&dev));
  KB_HIP(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
  // launch shape: 1024 x 2 (more, narrower threads: four wavefronts per SIMD
  // instead of two) on every level of rows of 1025..2048 states, where it
  // measured faster on every level (config 3: 1.77 vs 1.96 ms); on shorter
  // rows 512 x 4 on levels with at least two rows per workgroup slot and
  // 1024 x 2 on the smaller ones; KB_BWD_VARIANT=0 / 2 forces one shape
  // everywhere
  const char* vv = getenv("KB_BWD_VARIANT");
  const int variant = (vv && vv[0] == '2') ? 2 : (vv && vv[0] == '0') ? 0 : 1;
  // rows of 2049..8192 states: the low-register kernel (KB_BWD_LARGE=0: the
  // general row kernel; =2: also rows of 1025..2048 states)
  const char* lv = getenv("KB_BWD_LARGE");
  const int large = (lv && lv[0] == '0') ? 0 : (lv && lv[0] == '2') ? 2 : 1;
  int nb_max = std::max(1, n_cu * kb::bwd_blocks_per_cu(S, use_col, variant, large));
  // KB_BWD_GRID=n caps the persistent grid at n workgroups (tests: every
  // workgroup then walks many rows of a level)
  const char* gv = getenv("KB_BWD_GRID");
  if (gv && atoi(gv) > 0) nb_max = std::min(nb_max, atoi(gv));
  p->b_variant = variant;
  p->b_large = large;
  // owner-major constants of the low-register kernel (allocated once, when it first runs)
  if (kb::kb_use_large(S, large) && !p->b_om_const) {
    const size_t n_om = (size_t)kb::KB_OM_CONSTS * kb::kb_large_ld(S);
    if (alloc(&p->b_om_const, n_om)) return KB_ERR_HIP;
    p->owned.push_back(p->b_om_const);
    KB_HIP(hipMemset(p->b_om_const, 0, n_om * sizeof(float)));
  }
  if (p->b_contrib && p->b_nb_max == nb_max && p->b_slot == bwd_slot_floats(S, large)) return 0;
  p->b_slot = bwd_slot_floats(S, large);
  p->b_nb_max = nb_max;
  // one persistent bucket slot per workgroup of the per-level grids; kb_solve's
  // early launches use a second set, so slots for 2 nb_max are allocated
  p->b_n_partials = nb_max;
  if (p->b_contrib) {
    (void)hipFree(p->b_contrib);
    (void)hipFree(p->b_partial);
    for (auto& ptr : p->owned)
      if (ptr == (void*)p->b_contrib || ptr == (void*)p->b_partial) ptr = nullptr;
    p->b_contrib = nullptr;
    p->b_partial = nullptr;
    int rc = 0;
    rc |= alloc(&p->b_contrib, (size_t)2 * std::max(1, p->b_n_partials) * p->b_slot);
    rc |= alloc(&p->b_partial, (size_t)kb::reduce_chunks(2 * std::max(1, p->b_n_partials)) * 8 * S);
    p->owned.push_back(p->b_contrib);
    p->owned.push_back(p->b_partial);
    return rc ? KB_ERR_HIP : 0;
  }
  const int64_t NS = p->n_splits;
  int rc = 0;
  rc |= alloc(&p->b_staging, (size_t)std::max<int64_t>(1, 2 * NS) * kb::kb_stage_ld(S) + kb::KB_STAGE_TAIL);
  rc |= alloc(&p->b_split_on, (size_t)std::max<int64_t>(1, NS));
  rc |= alloc(&p->b_mask, (size_t)std::max(1, C));
  rc |= alloc(&p->b_rhs0, (size_t)std::max(1, C > 0 ? p->level_ptr[1] : 1) * S);
  rc |= alloc(&p->b_rhsc, (size_t)std::max(1, p->n_cls0) * S);
  rc |= alloc(&p->b_m_mask, (size_t)std::max(1, C > 0 ? p->level_ptr[1] : 1));
  rc |= alloc(&p->b_cls_active, (size_t)std::max(1, p->n_cls0));
  rc |= alloc(&p->b_ck_any, (size_t)std::max(1, p->n_chunks0));
  rc |= alloc(&p->b_contrib, (size_t)2 * std::max(1, p->b_n_partials) * p->b_slot);
  rc |= alloc(&p->b_partial, (size_t)kb::reduce_chunks(2 * std::max(1, p->b_n_partials)) * 8 * S);
  rc |= alloc(&p->b_acc, (size_t)8 * S);
  rc |= alloc(&p->b_work, (size_t)kb::epilogue_work_vectors() * S);
  rc |= alloc(&p->b_status, 2);
  rc |= alloc(&p->b_DL, S);
  rc |= alloc(&p->b_SL1, S);
  rc |= alloc(&p->b_SL2, S);
  rc |= alloc(&p->b_pS, S);
  rc |= alloc(&p->b_pD, S);
  rc |= alloc(&p->b_Ebar, S);
  rc |= alloc(&p->b_E, S);
  rc |= alloc(&p->b_mt, S);
  rc |= alloc(&p->b_col, S);
  for (void* ptr : {(void*)p->b_Ebar, (void*)p->b_E, (void*)p->b_mt, (void*)p->b_col,
                    (void*)p->b_staging, (void*)p->b_split_on, (void*)p->b_mask, (void*)p->b_contrib,
                    (void*)p->b_rhs0, (void*)p->b_rhsc, (void*)p->b_cls_active, (void*)p->b_ck_any, (void*)p->b_m_mask,
                    (void*)p->b_partial, (void*)p->b_acc, (void*)p->b_work, (void*)p->b_status, (void*)p->b_DL,
                    (void*)p->b_SL1, (void*)p->b_SL2, (void*)p->b_pS, (void*)p->b_pD})
    p->owned.push_back(ptr);
  return rc ? KB_ERR_HIP : 0;
}

// The backward in three parts (kb_backward runs them in order): checks, work
// buffers, constants, the row kernels' parameters and the zeroed bucket slots
// (`sets` sets of b_nb_max slots: 1, or 2 for kb_solve's early rows); one
// launch over rows [first, first + n) of level d on up to `grid` workgroups
// whose slots start at `poff`; the slot reduction, E adjoint and VJP epilogue.
// extra: workgroup slots beyond the first set that launches will add into
// (kb_solve's early launches), zeroed here as well
static int backward_setup(kb_plan* p, const kb_backward_io* io, hipStream_t st, kb::BwdParams& B, int extra) {
  if (!p || !io) return set_error(KB_ERR_ARG, "null argument");
  if (io->neumann_terms < 0) return set_error(KB_ERR_ARG, "neumann_terms must be non-negative");
  if (io->bicgstab_max_iter < 1) return set_error(KB_ERR_ARG, "max_iter must be at least 1");
  if (!(io->bicgstab_tol > 0.0)) return set_error(KB_ERR_ARG, "tol must be positive");
  if (!(io->bicgstab_breakdown_tol > 0.0)) return set_error(KB_ERR_ARG, "breakdown_tol must be positive");
  if (io->pruning_threshold < 0.0) return set_error(KB_ERR_ARG, "adjoint_pruning_threshold must be non-negative");
  if (!(io->neumann_rtol >= 0.0 && io->neumann_rtol < 1.0))
    return set_error(KB_ERR_ARG, "neumann_rtol must be in [0, 1)");
  int rc = ensure_backward_work(p, io->use_col_weights);
  if (rc) return rc;
  const int S = p->S;

  kb::BwdConstArgs K{};
  K.S = S;
  K.statewise = io->statewise;
  K.log_pS = io->log_pS;
  K.log_pD = io->log_pD;
  K.E = io->E;
  K.E_s1 = io->E_s1;
  K.E_s2 = io->E_s2;
  K.pre = p->d_pre;
  K.Ebar = io->Ebar;
  K.mt = io->max_coupling;
  K.col = io->col_log_probs;
  K.Ebar_pre = p->b_Ebar;
  K.E_pre = p->b_E;
  K.mt_pre = p->b_mt;
  K.col_pre = p->b_col;
  K.DL = p->b_DL;
  K.SL1 = p->b_SL1;
  K.SL2 = p->b_SL2;
  K.pS_state = p->b_pS;
  K.pD_state = p->b_pD;
  K.om = kb::kb_use_large(S, p->b_large) ? p->b_om_const : nullptr;
  // the same launch zeroes the bucket slots the launches will add into
  const size_t n_slots = (size_t)p->b_n_partials + std::min(std::max(extra, 0), p->b_n_partials);
  K.zero = p->b_contrib;
  K.n_zero = n_slots * p->b_slot;
  kb::launch_bwd_consts(K, st);

  B = kb::BwdParams{};
  B.tr = p->tree();
  B.S = S;
  B.n_terms = io->neumann_terms;
  B.rtol = (float)io->neumann_rtol;
  B.terms_out = io->neumann_terms_out;
  B.thr = (float)io->pruning_threshold;
  B.use_pruning = io->use_pruning;
  B.use_col = io->use_col_weights;
  B.pre = p->predev();
  B.DL = p->b_DL;
  B.Ebar = p->b_Ebar;
  B.E = p->b_E;
  B.SL1 = p->b_SL1;
  B.SL2 = p->b_SL2;
  B.mt = p->b_mt;
  B.col = p->b_col;
  B.pD = p->b_pD;
  B.pS = p->b_pS;
  B.pi = io->pi;
  B.pibar = io->pibar;
  B.rowmax = io->pibar_row_max;
  B.leaf_state = p->d_leaf;
  B.root_index = p->d_root_index;
  B.split_ptr = p->d_split_ptr;
  B.split_l = p->d_split_l;
  B.split_r = p->d_split_r;
  B.split_lsp = p->d_split_lsp;
  B.child_ptr = p->d_child_ptr;
  B.child_in = p->d_child_in;
  B.bslot = p->d_bslot;
  B.staging = p->b_staging;
  B.split_on = p->b_split_on;
  B.mask = io->active_mask ? (unsigned char*)io->active_mask : p->b_mask;
  B.contrib = p->b_contrib;
  B.sched_rows = p->d_sched_rows;
  B.row_kind = p->d_row_kind;
  B.variant = p->b_variant;
  B.large = p->b_large;
  B.om_tab = p->d_om_tab;
  B.om_const = p->b_om_const;
  B.rhs0 = p->b_rhs0;
  B.n_chunks0 = p->n_chunks0;
  B.ck_ptr = p->d_ck_ptr;
  B.cls_ck_ptr = p->d_cls_ck_ptr;
  B.ck_any = p->b_ck_any;
  B.rhsc = p->b_rhsc;
  B.m_side_ptr = p->d_m_side_ptr;
  B.m_side = p->d_m_side;
  B.m_root = p->d_m_root;
  B.m_mask = p->b_m_mask;
  B.cls_active = p->b_cls_active;
  // reuse the forward's split terms only for the outputs of the current forward
  const bool reuse = io->forward_token != 0 && io->forward_token == p->fwd_token && io->pi == p->fwd_pi &&
                     io->pibar == p->fwd_pibar;
  B.dts_in = reuse ? p->d_dts : nullptr;
  B.rep_of = p->d_rep_of;
  B.cls_ptr = p->d_cls_ptr;
  B.cls_rows = p->d_cls_rows;
  KB_HIP(hipGetLastError());
  return 0;
}

static int backward_level(kb_plan* p, kb::BwdParams& B, int d, int first, int n, int grid, int poff, hipStream_t st) {
  const int S = p->S;
  if (p->prof) KB_HIP(hipEventRecord(p->ev_bwd[2 * d], st));
  // level 0 (rows without splits) runs by class: one adjoint solve per class of identical rows
  B.class_mode = d == 0 ? 1 : 0;
  if (d == 0) kb::launch_bwd_level0_prep(B, p->level_ptr[1], p->n_cls0, st);
  B.variant = p->b_variant == 1 ? ((S > 1024 || n < 2 * grid) ? 2 : 0) : p->b_variant;
  kb::launch_bwd_wave(B, first, n, std::min(n, grid), poff, st);
  if (p->prof) KB_HIP(hipEventRecord(p->ev_bwd[2 * d + 1], st));
  return 0;
}

static int backward_finish(kb_plan* p, const kb_backward_io* io, int n_partials, hipStream_t st) {
  const int S = p->S;
  KB_HIP(hipGetLastError());
  kb::launch_bwd_reduce(p->b_contrib, n_partials, S, p->b_slot, kb::kb_slot_ld(S, p->b_large), p->b_partial,
                        p->d_pre, p->b_acc, st);
  KB_HIP(hipGetLastError());
  if (io->acc_out)
    KB_HIP(hipMemcpyAsync(io->acc_out, p->b_acc, (size_t)8 * S * sizeof(double), hipMemcpyDeviceToDevice, st));

  kb::EpiParams X{};
  X.tr = p->tree();
  X.ts = p->tscan();
  X.pd = p->predev();
  X.S = S;
  X.n_tlevels = p->n_tlevels;
  X.tlevel_ptr = p->d_tlevel_ptr;
  X.tlevel_node = p->d_tlevel_node;
  X.E = io->E;
  X.log_pS = io->log_pS;
  X.log_pD = io->log_pD;
  X.log_pL = io->log_pL;
  X.mt = io->max_coupling;
  X.col = io->col_log_probs;
  X.statewise = io->statewise;
  X.use_col = io->use_col_weights;
  X.theta = io->theta;
  X.col_weights = io->col_weights;
  X.acc = p->b_acc;
  X.n_fam = p->n_fam;
  X.n_items_rows = 1;
  X.max_iter = io->bicgstab_max_iter;
  X.tol = io->bicgstab_tol;
  X.breakdown = io->bicgstab_breakdown_tol;
  X.grad_theta = io->grad_theta;
  X.grad_col = io->grad_col;
  X.work = p->b_work;
  X.status = p->b_status;
  kb::launch_epilogue(X, st);
  KB_HIP(hipGetLastError());
  return 0;
}

static int level_rows(const kb_plan* p, int d) { return d == 0 ? p->n_cls0 : p->level_ptr[d + 1] - p->level_ptr[d]; }

extern "C" int kb_backward(kb_plan* p, const kb_backward_io* io, void* stream) {
  hipStream_t st = (hipStream_t)stream;
  kb::BwdParams B{};
  int rc = backward_setup(p, io, st, B, 0);
  for (int d = p ? p->n_levels - 1 : -1; !rc && d >= 0; --d)
    rc = backward_level(p, B, d, p->level_ptr[d], level_rows(p, d), p->b_nb_max, 0, st);
  return rc ? rc : backward_finish(p, io, p->b_n_partials, st);
}

extern "C" int kb_solve(kb_plan* p, const kb_forward_io* fio, const kb_backward_io* bio, void* stream) {
  if (!p || !fio || !bio) return set_error(KB_ERR_ARG, "null argument");
  if (bio->pi != fio->pi || bio->pibar != fio->pibar || bio->pibar_row_max != fio->pibar_row_max ||
      bio->E != fio->E || bio->Ebar != fio->Ebar || bio->E_s1 != fio->E_s1 || bio->E_s2 != fio->E_s2 ||
      bio->log_pS != fio->log_pS || bio->log_pD != fio->log_pD || bio->log_pL != fio->log_pL ||
      bio->max_coupling != fio->max_coupling || bio->col_log_probs != fio->col_log_probs)
    return set_error(KB_ERR_ARG, "kb_solve: the backward must read the forward's outputs");
  hipStream_t st = (hipStream_t)stream;
  kb::FwdParams F{};
  int rc = forward_setup(p, fio, st, F);
  if (rc) return rc;
  const int cut = p->overlap_cut;
  const int L = p->n_levels;
  // nothing to overlap, or per-launch timing on (its events time one launch per
  // level on one stream): the two passes one after the other
  if (cut < 1 || L < 3 || p->prof) {
    for (int d = 0; !rc && d < L; ++d) rc = forward_level(p, F, d, st);
    if (!rc) rc = forward_finish(p, fio, st);
    if (rc) return rc;
    kb_backward_io b2 = *bio;
    b2.forward_token = p->fwd_token;
    return kb_backward(p, &b2, stream);
  }
  kb_backward_io b2 = *bio;
  b2.forward_token = p->fwd_token;
  kb::BwdParams B{};
  // the early rows' workgroups use slots b_nb_max .. b_nb_max + overlap_grid - 1
  rc = backward_setup(p, &b2, st, B, p->overlap_grid);
  if (rc) return rc;
  if (!p->s2) {
    KB_HIP(hipStreamCreateWithFlags(&p->s2, hipStreamNonBlocking));
    KB_HIP(hipEventCreateWithFlags(&p->ev_fork, hipEventDisableTiming));
    KB_HIP(hipEventCreateWithFlags(&p->ev_join, hipEventDisableTiming));
  }
  // workgroups of the early launches: the rest of the CUs stay free for the
  // forward's narrow levels that run beside them
  const int eg = std::max(1, std::min(p->b_nb_max, p->overlap_grid));
  const int low = p->overlap_low;
  for (int d = 0; !rc && d <= cut; ++d) rc = forward_level(p, F, d, st);
  if (rc) return rc;
  KB_HIP(hipEventRecord(p->ev_fork, st));
  KB_HIP(hipStreamWaitEvent(p->s2, p->ev_fork, 0));
  kb::BwdParams B2 = B;
  for (int d = cut; !rc && d >= low; --d)
    if (p->n_early[d] > 0) rc = backward_level(p, B2, d, p->level_ptr[d], p->n_early[d], eg, p->b_nb_max, p->s2);
  if (rc) return rc;
  KB_HIP(hipEventRecord(p->ev_join, p->s2));
  for (int d = cut + 1; !rc && d < L; ++d) rc = forward_level(p, F, d, st);
  if (!rc) rc = forward_finish(p, fio, st);
  // the late rows down to the window's lowest level, then the levels below it whole
  for (int d = L - 1; !rc && d >= low; --d) {
    const int ne = d <= cut ? p->n_early[d] : 0, n = level_rows(p, d) - ne;
    if (n > 0) rc = backward_level(p, B, d, p->level_ptr[d] + ne, n, p->b_nb_max, 0, st);
  }
  if (rc) return rc;
  KB_HIP(hipStreamWaitEvent(st, p->ev_join, 0));
  for (int d = low - 1; !rc && d >= 0; --d) rc = backward_level(p, B, d, p->level_ptr[d], level_rows(p, d), p->b_nb_max, 0, st);
  return rc ? rc : backward_finish(p, &b2, p->b_nb_max + eg, st);
}

extern "C" {

int kb_e_adjoint(kb_plan* p, const kb_e_adjoint_io* io, void* stream) {
  if (!p || !io) return set_error(KB_ERR_ARG, "null argument");
  if (!io->E || !io->log_pS || !io->log_pD || !io->log_pL || !io->max_coupling || !io->col_log_probs || !io->acc ||
      !io->g_out || !io->work || !io->status)
    return set_error(KB_ERR_ARG, "null argument");
  if (io->bicgstab_max_iter < 1) return set_error(KB_ERR_ARG, "max_iter must be at least 1");
  if (!(io->bicgstab_tol > 0.0)) return set_error(KB_ERR_ARG, "tol must be positive");
  if (!(io->bicgstab_breakdown_tol > 0.0)) return set_error(KB_ERR_ARG, "breakdown_tol must be positive");
  if (kb::epilogue_work_vectors() > KB_E_ADJOINT_WORK_VECTORS)
    return set_error(KB_ERR_HIP, "the epilogue needs %d work vectors", kb::epilogue_work_vectors());
  kb::EpiParams X{};
  X.tr = p->tree();
  X.ts = p->tscan();
  X.pd = p->predev();
  X.S = p->S;
  X.n_tlevels = p->n_tlevels;
  X.tlevel_ptr = p->d_tlevel_ptr;
  X.tlevel_node = p->d_tlevel_node;
  X.E = io->E;
  X.log_pS = io->log_pS;
  X.log_pD = io->log_pD;
  X.log_pL = io->log_pL;
  X.mt = io->max_coupling;
  X.col = io->col_log_probs;
  X.statewise = io->statewise;
  X.use_col = io->use_col_weights;
  X.acc = io->acc;
  X.n_fam = p->n_fam;
  X.n_items_rows = 1;
  X.max_iter = io->bicgstab_max_iter;
  X.tol = io->bicgstab_tol;
  X.breakdown = io->bicgstab_breakdown_tol;
  X.work = io->work;
  X.status = io->status;
  X.q_extra = io->q_extra;
  X.no_norm = io->with_norm ? 0 : 1;
  X.w_out = io->w_out;
  X.g_out = io->g_out;
  kb::launch_epilogue(X, (hipStream_t)stream);
  KB_HIP(hipGetLastError());
  return 0;
}

int64_t kb_forward_token(const kb_plan* p) { return p ? p->fwd_token : 0; }

int kb_backward_stats(kb_plan* p, int32_t* n_iter, void* stream) {
  if (!p) return set_error(KB_ERR_ARG, "null argument");
  if (!p->b_status) return set_error(KB_ERR_ARG, "no backward has run on this plan");
  if (!p->h_status) KB_HIP(hipHostMalloc((void**)&p->h_status, 2 * sizeof(int), hipHostMallocDefault));
  KB_HIP(hipMemcpyAsync(p->h_status, p->b_status, 2 * sizeof(int), hipMemcpyDeviceToHost, (hipStream_t)stream));
  KB_HIP(hipStreamSynchronize((hipStream_t)stream));
  const int st[2] = {p->h_status[0], p->h_status[1]};
  if (n_iter) *n_iter = st[0];
  if (st[1])
    return set_error(KB_ERR_SOLVE, "E-adjoint BiCGSTAB solve failed after %d iterations", st[0]);
  return 0;
}

int kb_profile_enable(kb_plan* p, int enable) {
  if (!p) return set_error(KB_ERR_ARG, "null argument");
  if (enable && p->ev_fwd.empty()) {
    p->ev_fwd.resize(2 * (size_t)std::max(1, p->n_levels));
    p->ev_bwd.resize(2 * (size_t)std::max(1, p->n_levels));
    for (auto& e : p->ev_fwd) KB_HIP(hipEventCreate(&e));
    for (auto& e : p->ev_bwd) KB_HIP(hipEventCreate(&e));
  }
  p->prof = enable ? 1 : 0;
  return 0;
}

int kb_profile_read(kb_plan* p, int which, float* ms, int n) {
  if (!p || !ms) return set_error(KB_ERR_ARG, "null argument");
  if (p->ev_fwd.empty()) return set_error(KB_ERR_ARG, "profiling was never enabled on this plan");
  std::vector<hipEvent_t>& ev = which == 0 ? p->ev_fwd : p->ev_bwd;
  for (int w = 0; w < n && w < p->n_levels; ++w) {
    KB_HIP(hipEventSynchronize(ev[2 * w + 1]));
    KB_HIP(hipEventElapsedTime(&ms[w], ev[2 * w], ev[2 * w + 1]));
  }
  return 0;
}

int kb_forward_stats(kb_plan* p, int32_t* n_e_iter, double* loss64, void* stream) {
  if (!p) return set_error(KB_ERR_ARG, "null argument");
  KB_HIP(hipStreamSynchronize((hipStream_t)stream));
  if (n_e_iter) KB_HIP(hipMemcpy(n_e_iter, p->n_e_iter, sizeof(int), hipMemcpyDeviceToHost));
  if (loss64) KB_HIP(hipMemcpy(loss64, p->loss64, sizeof(double), hipMemcpyDeviceToHost));
  return 0;
}

}  // extern "C"
