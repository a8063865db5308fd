// Device kernels of the label-filtered Vamana build ("canonical_v2" release
// path of /root/reference/src/gpu_vamana_filtered.cu) for gfx950.
//
// Work decomposition (one wave64 each):
//   k_task_search   one (row, label) task: exact-label search, pool <= 32
//   k_row           one row: union-label search (pool <= 64) -> merge of the
//                   row's task results, old neighbours and union results ->
//                   label-quota compaction -> missing distances ->
//                   FilteredRobustPrune into the forward graph
//   k_csr           one row of the exact reverse CSR: forward row plus new
//                   reverse sources -> distances -> FilteredRobustPrune
// Candidate pools live in VGPRs (slot s = lane s); merged lists of <= 128
// entries live in two VGPRs per lane (entry i = lane i % 64, slot i / 64).
// Distances use the octet scheme of wave.h (canonical, bit-exact with the
// CPU oracle).
//
// The visited cache of the searches is a forgetful direct-mapped table in
// LDS. It is transparent: a repeated candidate has the same distance, so a
// duplicate insert into the canonical pool is a no-op, and once the pool is
// full its worst (distance, id) only falls, so a candidate rejected or evicted
// earlier is rejected again. Label filters are deterministic and every
// unfiltered insertion (entry points, posting seeds) precedes the filtered
// traversal, so skipping a cached id never changes the pool.
#pragma once

#include "locality.h"
#include "wave.h"

namespace dance {
namespace filt {

constexpr uint32_t kVisBits = 10;
constexpr uint32_t kVis = 1u << kVisBits;
constexpr uint32_t kWaves = 4;
constexpr uint32_t kBlock = 64 * kWaves;
constexpr uint32_t kMaxWorkC = 128;
constexpr uint32_t kCsrSlots = 4;  // CSR candidate lists up to 256 entries stay in VGPRs
constexpr uint32_t kCsrRegMax = 64u * kCsrSlots;
constexpr uint32_t kRandomAttempts = 1u << 20;
// LDS words per wave: visited cache + one distance batch (ids, distances).
constexpr uint32_t kSearchLds = kVis + 128u;
// LDS words per wave of k_csr: forward row + one distance batch.
constexpr uint32_t kCsrLds = 64u + 128u;
// Candidate lists longer than kCsrRegMax are pruned by k_csr_long, one
// workgroup of kLongWaves waves per row.
constexpr uint32_t kLongWaves = 16;
constexpr uint32_t kLongBlock = 64u * kLongWaves;
// Long rows that fit one key window use workgroups of this many waves.
constexpr uint32_t kLongSmallWaves = 4;

// Device counters (u64 each).
enum : uint32_t {
  kTaskDist = 0,
  kUnionDist,
  kWorkDist,
  kPruneDist,
  kCsrDist,
  kCsrPruneDist,
  kMergedCands,
  kQuotaDropped,
  kTouchedRows,
  kCsrCandidates,
  kBigRows,
  kBigMax,
  kPubDist,
  kPubTouched,
  kTaskExp,
  kTaskLab,
  kUnionExp,
  kUnionLab,
  kNumCounters
};
// Counters are striped over kCtrStripes copies (by workgroup) so that per-wave
// atomics do not serialise on one address; the host sums the stripes.
constexpr uint32_t kCtrStripes = 64;
__device__ __forceinline__ unsigned long long* ctr_at(unsigned long long* base, uint32_t idx) {
  return base + (size_t)(blockIdx.x & (kCtrStripes - 1u)) * kNumCounters + idx;
}

struct Labels {
  const uint32_t* off;     // N+1: point -> label list offsets
  const uint32_t* lab;     // label ids per point (sorted, unique)
  const uint32_t* lpo;     // num_labels+1: label -> posting offsets
  const uint32_t* lpts;    // postings (points per label, ascending)
  const uint32_t* starts;  // num_labels: label entry points
  uint32_t num_labels, universal;
  // Per point, its first 8 labels padded with DANCE_INV (two uint4), or the
  // marker {DANCE_INV, 0, ...} for points whose list the table cannot hold
  // (more than 8 labels, or the label DANCE_INV): membership tests then read
  // one 32-byte row instead of walking the list. nullptr: list walks only.
  const uint4* lab8;
  // Per point, a 32-bit label signature: bit sig_bit(l) set for each label l
  // of the point. A clear bit proves the label absent; a set bit leaves the
  // answer to the exact test.
  const uint32_t* sig;
};

__device__ __forceinline__ uint32_t sig_bit(uint32_t label) { return (label * 0x9E3779B1u) >> 27; }

// Builds Labels::lab8 (nullptr: skipped) and Labels::sig (one thread per point).
static __global__ void k_lab8(uint32_t N, const uint32_t* __restrict__ off, const uint32_t* __restrict__ lab,
                              uint4* __restrict__ lab8, uint32_t* __restrict__ sig) {
  const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= N) return;
  const uint32_t b = off[p], n = off[p + 1] - b;
  uint32_t sg = 0u;
  for (uint32_t i = 0; i < n; ++i) sg |= 1u << sig_bit(lab[b + i]);
  sig[p] = sg;
  if (!lab8) return;
  uint32_t v[8];
  bool fits = n <= 8;
#pragma unroll
  for (uint32_t i = 0; i < 8; ++i) {
    v[i] = (fits && i < n) ? lab[b + i] : DANCE_INV;
    if (fits && i < n && v[i] == DANCE_INV) fits = false;
  }
  if (!fits) {
    v[0] = DANCE_INV;
    v[1] = 0u;
  }
  lab8[2 * (size_t)p] = make_uint4(v[0], v[1], v[2], v[3]);
  lab8[2 * (size_t)p + 1] = make_uint4(v[4], v[5], v[6], v[7]);
}

// Point p's table row; false when p's list must be walked instead.
__device__ __forceinline__ bool lab8_row(const Labels& L, uint32_t p, uint4& a, uint4& b) {
  if (!L.lab8) return false;
  a = L.lab8[2 * (size_t)p];
  b = L.lab8[2 * (size_t)p + 1];
  return !(a.x == DANCE_INV && a.y == 0u);
}
__device__ __forceinline__ bool lab8_has(const uint4& a, const uint4& b, uint32_t label) {
  return label != DANCE_INV && (a.x == label || a.y == label || a.z == label || a.w == label || b.x == label ||
                                b.y == label || b.z == label || b.w == label);
}

struct Graph {
  uint32_t N, R;
  const uint32_t* g;  // N x R
  const uint32_t* d;  // N
  // Optional, N x R: the label signature (Labels::sig) of each entry's
  // point, read with the row so that label filters reject most neighbours
  // without a per-candidate label read (k_graph_sig).
  const uint32_t* sig = nullptr;
};

// Graph::sig of a graph: entry i of row r = sig[g[r][i]] for i < min(d[r], R)
// and valid ids, else 0 (one thread per entry).
static __global__ void k_graph_sig(uint32_t N, uint32_t R, const uint32_t* __restrict__ g,
                                   const uint32_t* __restrict__ d, const uint32_t* __restrict__ sig,
                                   uint32_t* __restrict__ out) {
  const uint64_t t = (uint64_t)grid_block() * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)N * R) return;
  const uint32_t r = (uint32_t)(t / R), i = (uint32_t)(t % R);
  const uint32_t id = g[t];
  out[t] = (i < min(d[r], R) && id < N) ? sig[id] : 0u;
}

// point_has_exact_label_device (gpu_vamana_filtered.cu:557-573)
__device__ __forceinline__ bool has_exact(const Labels& L, uint32_t p, uint32_t label) {
  uint4 a, b;
  if (label != DANCE_INV && lab8_row(L, p, a, b)) return lab8_has(a, b, label);
  const uint32_t e = L.off[p + 1];
  for (uint32_t i = L.off[p]; i < e; ++i) {
    const uint32_t v = L.lab[i];
    if (v == label) return true;
    if (v > label) break;
  }
  return false;
}

// has_common_label_device (gpu_vamana_filtered.cu:495-528); DANCE_INV as the
// universal label disables the universal rule.
__device__ __forceinline__ bool has_common(const Labels& L, uint32_t a, uint32_t b, uint32_t universal) {
  uint32_t i = L.off[a], j = L.off[b];
  const uint32_t ie = L.off[a + 1], je = L.off[b + 1];
  while (i < ie && j < je) {
    const uint32_t x = L.lab[i], y = L.lab[j];
    if (x == universal || y == universal || x == y) return true;
    if (x < y)
      ++i;
    else
      ++j;
  }
  return false;
}

// Union-search compatibility (gpu_vamana_filtered.cu:4561-4566): cand carries
// one of the row's labels exactly.
__device__ __forceinline__ bool compatible(const Labels& L, uint32_t row, uint32_t cand) {
  const uint32_t e = L.off[row + 1];
  uint4 a, b;
  if (lab8_row(L, cand, a, b)) {
    for (uint32_t p = L.off[row]; p < e; ++p)
      if (lab8_has(a, b, L.lab[p])) return true;
    return false;
  }
  for (uint32_t p = L.off[row]; p < e; ++p)
    if (has_exact(L, cand, L.lab[p])) return true;
  return false;
}

// filtered_selected_covers_common_labels (include/filtered_label_coverage.cuh:7-44):
// every label shared by target and cand is also a label of selected.
__device__ __forceinline__ bool covers(const Labels& L, uint32_t target, uint32_t selected, uint32_t cand) {
  uint32_t ti = L.off[target], ci = L.off[cand];
  const uint32_t te = L.off[target + 1], ce = L.off[cand + 1];
  while (ti < te && ci < ce) {
    const uint32_t tl = L.lab[ti], cl = L.lab[ci];
    if (tl < cl) {
      ++ti;
    } else if (cl < tl) {
      ++ci;
    } else {
      if (!has_exact(L, selected, tl)) return false;
      ++ti;
      ++ci;
    }
  }
  return true;
}

// Bit q is set when c carries the row's q-th label (rows with <= 32 labels).
// For sorted unique label lists covers(row, s, c) == !(mask(c) & ~mask(s)):
// the labels shared by row and c are exactly the set bits of mask(c).
__device__ __forceinline__ uint32_t row_mask(const Labels& L, uint32_t row, uint32_t c) {
  uint4 a, b;
  if (lab8_row(L, c, a, b)) {
    uint32_t bits = 0;
    const uint32_t rb = L.off[row], re = L.off[row + 1];
    for (uint32_t q = 0; rb + q < re; ++q)
      if (lab8_has(a, b, L.lab[rb + q])) bits |= 1u << q;
    return bits;
  }
  uint32_t i = L.off[row], j = L.off[c], bits = 0, q = 0;
  const uint32_t ie = L.off[row + 1], je = L.off[c + 1];
  while (i < ie && j < je) {
    const uint32_t x = L.lab[i], y = L.lab[j];
    if (x == y) {
      bits |= 1u << q;
      ++i;
      ++q;
      ++j;
    } else if (x < y) {
      ++i;
      ++q;
    } else {
      ++j;
    }
  }
  return bits;
}
constexpr uint32_t kMaskLabels = 32;

// ---------------------------------------------------------------------------
// Canonical pool (gpu_vamana_filtered.cu:4156-4263): no early reject; the
// worst entry is the largest (distance, id); selection takes the smallest
// unexpanded (distance, id) with distance <= FLT_MAX.
// ---------------------------------------------------------------------------
struct CanonPool {
  uint32_t id;
  float d;
  uint32_t ex;
  uint32_t count, cap;
  int wpos;
  float wd;
  uint32_t wid;

  __device__ __forceinline__ void init(uint32_t c) {
    id = DANCE_INV;
    d = FLT_MAX;
    ex = 0;
    count = 0;
    cap = c;
    wpos = -1;
    wd = -FLT_MAX;
    wid = 0;
  }
  __device__ __forceinline__ void recompute_worst(uint32_t lane) {
    const bool v = lane < count && d == d;
    const int M = wave_max_i(v ? fkey(d) : INT_MIN);
    if (M == INT_MIN) {
      wpos = -1;
      wd = -FLT_MAX;
      wid = 0;
      return;
    }
    const bool tie = v && fkey(d) == M;
    const uint32_t W = wave_max_u(tie ? id : 0u);
    wpos = ffs64(wballot(tie && id == W));
    wd = __int_as_float(M);
    wid = W;
  }
  // One of: refresh a duplicate's distance, append, replace the worst. The
  // slot registers change by selects on one path, so the compiler does not
  // copy them at branch joins; only the worst recomputation branches.
  __device__ __forceinline__ void insert(uint32_t nid, float nd, uint32_t lane) {
    const uint64_t dm = wballot(lane < count && id == nid);
    const int dup = dm ? ffs64(dm) : -1;
    const bool refresh = dm != 0 && nd < rdlane_f(d, dup & 63);
    const bool append = dm == 0 && count < cap;
    const bool replace = dm == 0 && count >= cap && wpos >= 0 && (nd < wd || (nd == wd && nid < wid));
    const int pos = dm ? dup : (append ? (int)count : wpos);
    const bool hit = (refresh || append || replace) && (int)lane == pos;
    id = hit ? nid : id;  // a duplicate keeps its id
    d = hit ? nd : d;
    ex = hit ? 0u : ex;
    count += append ? 1u : 0u;
    if (refresh || append || replace) recompute_worst(lane);
  }
  // True when (nd, nid) is certainly rejected: the pool is full and the pair
  // is not below the worst entry (which only falls while the pool is full).
  __device__ __forceinline__ bool full_reject(float nd, uint32_t nid) const {
    return count >= cap && wpos >= 0 && !(nd < wd || (nd == wd && nid < wid));
  }
  __device__ __forceinline__ int select(uint32_t lane) const {
    const bool c = lane < count && ex == 0 && d <= FLT_MAX;
    const int M = wave_min_i(c ? fkey(d) : INT_MAX);
    if (M == INT_MAX) return -1;
    const bool tie = c && fkey(d) == M;
    const uint32_t I = wave_min_u(tie ? id : DANCE_INV);
    return ffs64(wballot(tie && id == I));
  }
};

// Search skeleton shared by the task search and the union search.
template <int DT, int CPL>
struct FSearch {
  RowSet rs;
  uint32_t N, row, lane, grp, sub;
  uint32_t* vis;
  uint32_t* lst;
  float* lsd;
  uint4 av[CPL];
  CanonPool P;
  uint32_t ndist;
  uint32_t nexp;  // adjacency rows read (uniform)

  __device__ __forceinline__ void init(const RowSet& rs_, uint32_t N_, uint32_t row_, uint32_t* lds, uint32_t cap) {
    rs = rs_;
    N = N_;
    row = row_;
    lane = lane_id();
    grp = lane >> 3;
    sub = lane & 7u;
    vis = lds;
    lst = lds + kVis;
    lsd = reinterpret_cast<float*>(lds + kVis + 64);
    ndist = 0;
    nexp = 0;
    for (uint32_t i = lane; i < kVis; i += 64) vis[i] = DANCE_INV;
    load_row<CPL>(rs, row, true, sub, av);
    P.init(cap);
    wave_sync();
  }

  // One batch of up to 64 candidates in insertion order (lane order; DANCE_INV
  // = no candidate). accept(c, sg) is the label filter of the current phase;
  // sg is c's label signature when the caller has it (a graph row with
  // signatures), else all ones (no information).
  template <typename F>
  __device__ __forceinline__ void batch(uint32_t c, F&& accept, uint32_t sg = 0xFFFFFFFFu) {
    const bool v = c < N && c != row;
    const uint32_t slot = (c * 0x9E3779B1u) >> (32 - kVisBits);
    const bool seen = v && vis[slot] == c;
    const bool need = v && !seen && accept(c, sg);
    const uint64_t m = wballot(need);
    if (m) {
      const uint32_t n = popc64(m);
      if (need) lst[mbcnt64(m)] = c;
      wave_sync();
      batch_dist<DT, CPL>(rs, av, lst, lsd, n, grp, sub);
      ndist += n;
      const uint32_t ck = lane < n ? lst[lane] : DANCE_INV;
      const float dk = lane < n ? lsd[lane] : FLT_MAX;
      uint64_t km = wballot(lane < n && !P.full_reject(dk, ck));
      while (km) {
        const int k = ffs64(km);
        km &= km - 1;
        P.insert(rdlane_u(ck, k), rdlane_f(dk, k), lane);
      }
    }
    if (v && !seen) vis[slot] = c;
    wave_sync();
  }

  template <typename F>
  __device__ __forceinline__ void neighbours(const Graph& G, uint32_t u, F&& accept) {
    const uint32_t deg = min(G.d[u], G.R);
    const size_t b = (size_t)u * G.R;
    ++nexp;
    for (uint32_t j = 0; j < deg; j += 64) {
      const bool in = j + lane < deg;
      batch(in ? G.g[b + j + lane] : DANCE_INV, accept, in && G.sig ? G.sig[b + j + lane] : 0xFFFFFFFFu);
    }
  }

  template <typename F>
  __device__ __forceinline__ void expand(const Graph& G, uint32_t steps, F&& accept) {
    for (uint32_t step = 0; step < steps; ++step) {
      const int pos = P.select(lane);
      if (pos < 0) break;
      if ((int)lane == pos) P.ex = 1;
      neighbours(G, rdlane_u(P.id, pos), accept);
    }
  }
};

// ---------------------------------------------------------------------------
// FilteredRobustPrune (canonical_exact_prune / canonical_exact_prune_csr,
// gpu_vamana_filtered.cu:4876-4994, 5130-5230) over a list held in VGPRs:
// entry e*64+lane is (id[e], d[e]); bit e of `rem` marks it removed or absent.
// Repeatedly selects the smallest (distance, id, index) and removes every
// remaining candidate c with covers(row, sel, c), D(sel, c) > 0 and
// alpha * D(sel, c) <= d(c). Lane k < R receives the k-th selected id.
// ---------------------------------------------------------------------------
template <int DT, int CPL, int E>
__device__ __forceinline__ uint32_t prune_regs(const RowSet& rs, const Labels& L, uint32_t row, uint32_t R,
                                               float alpha, const uint32_t (&id)[E], const float (&d)[E],
                                               uint32_t rem, uint32_t* lst, float* lsd, uint32_t lane,
                                               uint32_t& outv, uint32_t& ndist) {
  const uint32_t grp = lane >> 3, sub = lane & 7u;
  const bool use_mask = L.off[row + 1] - L.off[row] <= kMaskLabels;
  uint32_t msk[E];
#pragma unroll
  for (int e = 0; e < E; ++e) msk[e] = (use_mask && !((rem >> e) & 1u)) ? row_mask(L, row, id[e]) : 0u;
  uint32_t sel = 0;
  outv = DANCE_INV;
  while (sel < R) {
    int bk = INT_MAX;
    uint32_t bid = DANCE_INV, bix = DANCE_INV;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (!((rem >> e) & 1u) && d[e] <= FLT_MAX) {
        const int k = fkey(d[e]);
        if (k < bk || (k == bk && id[e] < bid)) {
          bk = k;
          bid = id[e];
          bix = (uint32_t)e * 64u + lane;
        }
      }
    }
    const int M = wave_min_i(bk);
    if (M == INT_MAX) break;
    const uint32_t I = wave_min_u(bk == M ? bid : DANCE_INV);
    const uint32_t X = wave_min_u(bk == M && bid == I ? bix : DANCE_INV);
    uint32_t mv = msk[0];
#pragma unroll
    for (int e = 1; e < E; ++e)
      if ((uint32_t)e == (X >> 6)) mv = msk[e];
    const uint32_t msel = rdlane_u(mv, (int)(X & 63u));
    if (lane == sel) outv = I;
    if (lane == (X & 63u)) rem |= 1u << (X >> 6);
    ++sel;
    uint4 bv[CPL];
    load_row<CPL>(rs, I, true, sub, bv);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const bool live = !((rem >> e) & 1u);
      const bool need = live && (use_mask ? (msk[e] & ~msel) == 0u : covers(L, row, I, id[e]));
      const uint64_t m = wballot(need);
      if (m) {
        const uint32_t n = popc64(m), pos = mbcnt64(m);
        if (need) lst[pos] = id[e];
        wave_sync();
        batch_dist<DT, CPL>(rs, bv, lst, lsd, n, grp, sub);
        ndist += n;
        if (need) {
          const float pd = lsd[pos];
          if (pd > 0.0f && alpha * pd <= d[e]) rem |= 1u << e;
        }
        wave_sync();
      }
    }
  }
  return sel;
}


// ---------------------------------------------------------------------------
// Kernels.
// ---------------------------------------------------------------------------

// filtered_deterministic_random_graph_kernel (gpu_vamana_filtered.cu:716-744):
// `target` distinct non-self neighbours from a hash stream. The attempt bound
// only guarantees termination; it is far above what any input needs.
static __global__ void k_random_graph(uint32_t N, uint32_t R, uint32_t target, uint32_t seed, uint32_t* g,
                                      uint32_t* deg) {
  const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= N) return;
  uint32_t* out = g + (size_t)row * R;
  uint32_t n = 0;
  for (uint32_t attempt = 0; n < target && attempt < kRandomAttempts; ++attempt) {
    const uint32_t c = d_hash_u32(row * 0x9e3779b1u ^ seed * 0x85ebca6bu ^ attempt * 0xc2b2ae35u) % N;
    if (c == row) continue;
    bool dup = false;
    for (uint32_t i = 0; i < n && !dup; ++i) dup = out[i] == c;
    if (!dup) out[n++] = c;
  }
  for (uint32_t i = n; i < R; ++i) out[i] = DANCE_INV;
  deg[row] = n;
}

// canonical_make_task_rows: task p (a position in the label array) -> its row.
// Task order from a row order: pos[k] = label count of row order[k] (pos[N]
// = 0, then an exclusive scan), and the tasks of row order[k] (its label
// positions off[r] .. off[r + 1]) at pos[k] .. (one thread per row).
static __global__ void k_task_counts(uint32_t N, const uint32_t* __restrict__ off, const uint32_t* __restrict__ order,
                                     uint32_t* __restrict__ pos) {
  const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k > N) return;
  pos[k] = k == N ? 0u : off[order[k] + 1] - off[order[k]];
}
static __global__ void k_task_fill(uint32_t N, const uint32_t* __restrict__ off, const uint32_t* __restrict__ order,
                                   const uint32_t* __restrict__ pos, uint32_t* __restrict__ torder) {
  const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= N) return;
  const uint32_t r = order[k], b = off[r], n = off[r + 1] - b, p = pos[k];
  for (uint32_t j = 0; j < n; ++j) torder[p + j] = b + j;
}

static __global__ void k_task_rows(uint32_t N, const uint32_t* off, uint32_t* task_rows) {
  const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= N) return;
  for (uint32_t p = off[row]; p < off[row + 1]; ++p) task_rows[p] = row;
}

// canonical_filtered_task_search (gpu_vamana_filtered.cu:4265-4426) with the
// posting anchor off: label entry point and <= 16 posting seeds (unfiltered),
// then the exact-label traversal; the first `keep` pool slots are the output.
template <int DT, int CPL>
__global__ __launch_bounds__(kBlock) void k_task_search(RowSet rs, Graph G, Labels L, const uint32_t* task_rows,
                                                        const uint32_t* order, uint32_t tasks, uint32_t cap,
                                                        uint32_t keep, uint32_t steps, uint32_t* out_ids,
                                                        float* out_d, unsigned long long* ctr) {
  extern __shared__ uint32_t smem[];
  const uint32_t w = wave_index();
  const uint32_t k = xcd_block(grid_block(), grid_blocks()) * kWaves + w;
  if (k >= tasks) return;
  const uint32_t t = order ? order[k] : k;  // order: a permutation of the tasks
  const uint32_t lane = lane_id();
  const uint32_t row = task_rows[t], label = L.lab[t];
  const uint32_t N = G.N;
  const size_t ob = (size_t)t * keep;
  if (row >= N || label >= L.num_labels || label == L.universal) {
    if (lane < keep) {
      out_ids[ob + lane] = DANCE_INV;
      out_d[ob + lane] = FLT_MAX;
    }
    return;
  }
  FSearch<DT, CPL> S;
  S.init(rs, N, row, smem + w * kSearchLds, cap);
  auto any = [](uint32_t, uint32_t) { return true; };
  const uint32_t lbit = 1u << sig_bit(label);
  uint32_t nlab = 0;  // per lane: label rows read
  auto exact = [&](uint32_t c, uint32_t sg) {
    const bool maybe = (sg & lbit) != 0u;
    nlab += maybe ? 1u : 0u;
    return maybe && has_exact(L, c, label);
  };
  S.batch(lane == 0 ? L.starts[label] : DANCE_INV, any);
  const uint32_t pb = L.lpo[label], pc = L.lpo[label + 1] - pb;
  const uint32_t sc = min(16u, pc);
  S.batch(lane < sc ? L.lpts[pb + d_hash_u32(row + lane * 7919u + label * 17u) % pc] : DANCE_INV, any);
  S.neighbours(G, row, exact);
  S.expand(G, steps, exact);
  if (lane < keep) {
    const bool h = lane < S.P.count;
    out_ids[ob + lane] = h ? S.P.id : DANCE_INV;
    out_d[ob + lane] = h ? S.P.d : FLT_MAX;
  }
  if (ctr) {
    const uint32_t lab = wave_sum_u(nlab);
    if (lane == 0) {
      atomicAdd(ctr_at(ctr, kTaskDist), (unsigned long long)S.ndist);
      atomicAdd(ctr_at(ctr, kTaskExp), (unsigned long long)S.nexp);
      atomicAdd(ctr_at(ctr, kTaskLab), (unsigned long long)lab);
    }
  }
}

struct RowArgs {
  uint32_t ocap, okeep, steps, global_start, C, tkeep;
  float alpha;
  const uint32_t* task_ids;
  const float* task_d;
  uint32_t* gout;  // N x R forward graph
  uint32_t* dout;  // N
  unsigned long long* ctr;
  const uint32_t* order;  // processing order of the rows (a permutation), or nullptr
};

// Merged candidate list of one row: entry i in lane i % 64, slot i / 64.
struct MList {
  uint32_t id0, id1;
  float d0, d1;
  uint32_t count;
  // canonical_merge_one_warp (gpu_vamana_filtered.cu:4672-4701): skip invalid,
  // self and overflow; a duplicate keeps the smaller distance; else append.
  __device__ __forceinline__ void merge_one(uint32_t c, float dist, uint32_t row, uint32_t N, uint32_t C,
                                            uint32_t lane) {
    if (c >= N || c == row || count >= C) return;
    const uint64_t m0 = wballot(lane < count && id0 == c);
    const uint64_t m1 = count > 64 ? wballot(lane + 64 < count && id1 == c) : 0ull;
    if (m0 | m1) {
      if (m0) {
        if ((int)lane == ffs64(m0) && dist < d0) d0 = dist;
      } else {
        if ((int)lane == ffs64(m1) && dist < d1) d1 = dist;
      }
      return;
    }
    if (lane == (count & 63u)) {
      if (count < 64) {
        id0 = c;
        d0 = dist;
      } else {
        id1 = c;
        d1 = dist;
      }
    }
    ++count;
  }
  // Runs merge_one over the lanes set in `m`, in lane order.
  __device__ __forceinline__ void merge_lanes(uint64_t m, uint32_t c, float dist, uint32_t row, uint32_t N,
                                              uint32_t C, uint32_t lane) {
    while (m && count < C) {
      const int k = ffs64(m);
      m &= m - 1;
      merge_one(rdlane_u(c, k), rdlane_f(dist, k), row, N, C, lane);
    }
  }
};

// One row of a canonical round: canonical_ordinary_search restricted to
// compatible candidates (gpu_vamana_filtered.cu:4529-4670),
// canonical_merge_candidates with the label quota (:4703-4842),
// canonical_compute_work_distances (:4844-4871) and canonical_exact_prune
// (:4876-4994) fused; the merged list never leaves the wave.
template <int DT, int CPL>
__global__ __launch_bounds__(kBlock) void k_row(RowSet rs, Graph G, Labels L, RowArgs A) {
  extern __shared__ uint32_t smem[];
  const uint32_t w = wave_index();
  const uint32_t k = xcd_block(grid_block(), grid_blocks()) * kWaves + w;
  const uint32_t N = G.N, R = G.R;
  if (k >= N) return;
  const uint32_t row = A.order ? A.order[k] : k;
  const uint32_t lane = lane_id();
  uint32_t* lds = smem + w * kSearchLds;
  const uint32_t lb = L.off[row], le = L.off[row + 1];

  // 1. union-label search: label entry points and posting seeds unfiltered,
  //    then the global start and the traversal restricted to compatible ids
  FSearch<DT, CPL> S;
  S.init(rs, N, row, lds, A.ocap);
  auto any = [](uint32_t, uint32_t) { return true; };
  const uint32_t rsig = L.sig ? L.sig[row] : 0xFFFFFFFFu;
  uint32_t nlab = 0;  // per lane: label rows read
  auto compat = [&](uint32_t c, uint32_t sg) {
    const bool maybe = (sg & rsig) != 0u;
    nlab += maybe ? 1u : 0u;
    return maybe && compatible(L, row, c);
  };
  for (uint32_t p = lb; p < le; ++p) {
    const uint32_t label = L.lab[p];
    if (label >= L.num_labels) continue;
    S.batch(lane == 0 ? L.starts[label] : DANCE_INV, any);
    const uint32_t pb = L.lpo[label], pc = L.lpo[label + 1] - pb;
    const uint32_t sc = min(64u, pc);
    S.batch(lane < sc ? L.lpts[pb + d_hash_u32(row + lane * 7919u + label * 17u) % pc] : DANCE_INV, any);
  }
  S.batch(lane == 0 ? A.global_start : DANCE_INV, compat);
  S.neighbours(G, row, compat);
  S.expand(G, A.steps, compat);
  const bool oh = lane < A.okeep && lane < S.P.count;
  const uint32_t o_id = oh ? S.P.id : DANCE_INV;
  const float o_d = oh ? S.P.d : FLT_MAX;
  uint32_t ndist_prune = 0, ndist_work = 0;
  const uint32_t ndist_union = S.ndist;
  const uint32_t nlab_union = A.ctr ? wave_sum_u(nlab) : 0u;

  // 2. merge: task results, old label-sharing neighbours, union results
  MList M;
  M.id0 = M.id1 = DANCE_INV;
  M.d0 = M.d1 = FLT_MAX;
  M.count = 0;
  const uint32_t C = A.C;
  {
    const size_t tb = (size_t)lb * A.tkeep, te = (size_t)le * A.tkeep;
    for (size_t b = tb; b < te && M.count < C; b += 64) {
      const bool in = b + lane < te;
      const uint32_t c = in ? A.task_ids[b + lane] : DANCE_INV;
      const float dd = in ? A.task_d[b + lane] : FLT_MAX;
      M.merge_lanes(wballot(c < N && c != row), c, dd, row, N, C, lane);
    }
    const uint32_t deg = min(G.d[row], R);
    const uint32_t c = lane < deg ? G.g[(size_t)row * R + lane] : DANCE_INV;
    const bool ok = c < N && c != row && has_common(L, row, c, DANCE_INV);
    M.merge_lanes(wballot(ok), c, FLT_MAX, row, N, C, lane);
    M.merge_lanes(wballot(o_id < N && o_id != row), o_id, o_d, row, N, C, lane);
  }

  // 3. label quota for rows with 1..16 labels: each candidate is assigned to
  //    its row label of smallest (cardinality, label id) that still has room;
  //    candidates with no such label are dropped; the order is kept.
  const uint32_t lc = le - lb;
  uint32_t count = M.count;
  if (lc >= 1 && lc <= 16) {
    uint32_t* rl = lds;        // row labels [16]
    uint32_t* rk = lds + 16;   // rank of row label q
    uint32_t* sid = lds + 64;  // compaction staging [128]
    float* sd = reinterpret_cast<float*>(lds + 192);
    const uint32_t myl = lane < lc ? L.lab[lb + lane] : DANCE_INV;
    const uint32_t myc = lane < lc ? (myl < L.num_labels ? L.lpo[myl + 1] - L.lpo[myl] : 0u) : DANCE_INV;
    // rank by (cardinality, label, position): equal to the reference's
    // first-minimum choice among the eligible labels
    uint32_t rank = 0;
    for (uint32_t q = 0; q < lc; ++q) {
      const uint32_t ql = rdlane_u(myl, q), qc = rdlane_u(myc, q);
      rank += (qc < myc || (qc == myc && (ql < myl || (ql == myl && q < lane)))) ? 1u : 0u;
    }
    if (lane < lc) {
      rl[lane] = myl;
      rk[lane] = rank;
    }
    wave_sync();
    uint32_t quota = (R + lc - 1) / lc;
    if (quota < A.tkeep) quota = A.tkeep;
    auto elig = [&](uint32_t c, bool valid) -> uint32_t {
      uint32_t bits = 0;
      if (valid)
        for (uint32_t q = 0; q < lc; ++q)
          if (has_exact(L, c, rl[q])) bits |= 1u << rk[q];
      return bits;
    };
    const uint32_t e0 = elig(M.id0, lane < count), e1 = elig(M.id1, lane + 64 < count);
    uint64_t cnt_lo = 0, cnt_hi = 0;  // 8-bit counters per rank (quota <= 64)
    uint32_t full = 0;
    uint64_t k0 = 0, k1 = 0;
    for (uint32_t i = 0; i < count; ++i) {
      const uint32_t e = rdlane_u(i < 64 ? e0 : e1, (int)(i & 63u)) & ~full;
      if (!e) continue;
      const uint32_t r = (uint32_t)__builtin_ctz(e);
      uint32_t v;
      if (r < 8) {
        cnt_lo += 1ull << (8 * r);
        v = (uint32_t)(cnt_lo >> (8 * r)) & 255u;
      } else {
        cnt_hi += 1ull << (8 * (r - 8));
        v = (uint32_t)(cnt_hi >> (8 * (r - 8))) & 255u;
      }
      if (v >= quota) full |= 1u << r;
      if (i < 64)
        k0 |= 1ull << i;
      else
        k1 |= 1ull << (i - 64);
    }
    const uint32_t kept = popc64(k0) + popc64(k1);
    if ((k0 >> lane) & 1ull) {
      sid[mbcnt64(k0)] = M.id0;
      sd[mbcnt64(k0)] = M.d0;
    }
    if ((k1 >> lane) & 1ull) {
      sid[popc64(k0) + mbcnt64(k1)] = M.id1;
      sd[popc64(k0) + mbcnt64(k1)] = M.d1;
    }
    wave_sync();
    M.id0 = lane < kept ? sid[lane] : DANCE_INV;
    M.d0 = lane < kept ? sd[lane] : FLT_MAX;
    M.id1 = lane + 64 < kept ? sid[lane + 64] : DANCE_INV;
    M.d1 = lane + 64 < kept ? sd[lane + 64] : FLT_MAX;
    wave_sync();
    if (A.ctr && lane == 0) atomicAdd(ctr_at(A.ctr, kQuotaDropped), (unsigned long long)(count - kept));
    count = kept;
  }

  // 4. distances of entries merged without one
  uint32_t* lst = lds + kVis;
  float* lsd = reinterpret_cast<float*>(lds + kVis + 64);
  uint32_t id[2] = {M.id0, M.id1};
  float d[2] = {M.d0, M.d1};
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const bool need = (uint32_t)e * 64u + lane < count && d[e] == FLT_MAX;
    const uint64_t m = wballot(need);
    if (m) {
      const uint32_t n = popc64(m), pos = mbcnt64(m);
      if (need) lst[pos] = id[e];
      wave_sync();
      batch_dist<DT, CPL>(rs, S.av, lst, lsd, n, S.grp, S.sub);
      ndist_work += n;
      if (need) d[e] = lsd[pos];
      wave_sync();
    }
  }

  // 5. FilteredRobustPrune into the forward graph
  uint32_t rem = 0;
  if (lane >= count) rem |= 1u;
  if (lane + 64 >= count) rem |= 2u;
  uint32_t outv;
  const uint32_t sel = prune_regs<DT, CPL, 2>(rs, L, row, R, A.alpha, id, d, rem, lst, lsd, lane, outv, ndist_prune);
  if (lane < R) A.gout[(size_t)row * R + lane] = lane < sel ? outv : DANCE_INV;
  if (lane == 0) {
    A.dout[row] = sel;
    if (A.ctr) {
      atomicAdd(ctr_at(A.ctr, kUnionDist), (unsigned long long)ndist_union);
      atomicAdd(ctr_at(A.ctr, kUnionExp), (unsigned long long)S.nexp);
      atomicAdd(ctr_at(A.ctr, kUnionLab), (unsigned long long)nlab_union);
      atomicAdd(ctr_at(A.ctr, kWorkDist), (unsigned long long)ndist_work);
      atomicAdd(ctr_at(A.ctr, kPruneDist), (unsigned long long)ndist_prune);
      atomicAdd(ctr_at(A.ctr, kMergedCands), (unsigned long long)count);
    }
  }
}

// canonical_reverse_count (gpu_vamana_filtered.cu:4996-5016): in-degree per
// target of the forward graph.
static __global__ void k_rev_count(uint32_t N, uint32_t R, const uint32_t* g, const uint32_t* deg,
                                   uint32_t* indeg) {
  const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= N) return;
  const uint32_t n = min(deg[row], R);
  for (uint32_t i = 0; i < n; ++i) {
    const uint32_t t = g[(size_t)row * R + i];
    if (t < N && t != row) atomicAdd(indeg + t, 1u);
  }
}

// canonical_reverse_fill (gpu_vamana_filtered.cu:5018-5034): sources grouped
// by target, in arbitrary order within a target (the prune's result does not
// depend on it: live candidate ids are unique).
static __global__ void k_rev_fill(uint32_t N, uint32_t R, const uint32_t* g, const uint32_t* deg,
                                  const uint32_t* roff, uint32_t* cursor, uint32_t* rids) {
  const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= N) return;
  const uint32_t n = min(deg[row], R);
  for (uint32_t i = 0; i < n; ++i) {
    const uint32_t t = g[(size_t)row * R + i];
    if (t < N && t != row) rids[roff[t] + atomicAdd(cursor + t, 1u)] = row;
  }
}

// Sizes of the candidate lists that exceed the VGPR capacity (they get
// global scratch); N+1 entries, the last one 0, ready for an exclusive scan.
static __global__ void k_big_sizes(uint32_t N, uint32_t R, const uint32_t* deg, const uint32_t* roff,
                                   uint32_t* big) {
  const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row > N) return;
  if (row == N) {
    big[N] = 0;
    return;
  }
  const uint32_t in = roff[row + 1] - roff[row];
  const uint32_t ub = min(deg[row], R) + in;
  big[row] = (in > 0 && ub > kCsrRegMax) ? ub : 0u;
}

struct CsrArgs {
  float alpha;
  const uint32_t* roff;  // N+1 reverse offsets
  const uint32_t* rids;  // reverse sources
  const uint32_t* boff;  // N+1 scratch offsets of long lists
  float* bd;
  uint8_t* brem;
  uint32_t* bmask;
  uint32_t* gout;
  uint32_t* dout;
  unsigned long long* ctr;
  uint32_t win;  // k_csr_long key-window target, 1 .. kLongList / 2
};

// canonical_reverse_candidate_count/fill, canonical_csr_candidate_distances
// and canonical_exact_prune_csr (gpu_vamana_filtered.cu:5036-5230) for one
// row. The candidate list is the forward row followed by the reverse sources
// not already in it; entry i is the i-th of that concatenation (duplicates
// are marked removed instead of compacted away, so live ids stay unique and
// the selection is unchanged). Rows without reverse sources keep their row;
// rows of more than kCsrRegMax candidates are left to k_csr_long.
template <int DT, int CPL>
__global__ __launch_bounds__(kBlock) void k_csr(RowSet rs, Graph G, Labels L, CsrArgs A) {
  extern __shared__ uint32_t smem[];
  const uint32_t w = wave_index();
  const uint32_t row = xcd_block(grid_block(), grid_blocks()) * kWaves + w;
  const uint32_t N = G.N, R = G.R;
  if (row >= N) return;
  const uint32_t lane = lane_id();
  const size_t gb = (size_t)row * R;
  const uint32_t s0 = A.roff[row], s1 = A.roff[row + 1];
  if (s0 == s1) {
    if (lane < R) A.gout[gb + lane] = G.g[gb + lane];
    if (lane == 0) A.dout[row] = G.d[row];
    return;
  }
  const uint32_t deg = min(G.d[row], R);
  const uint32_t n = deg + (s1 - s0);
  if (n > kCsrRegMax) return;
  uint32_t* fw = smem + w * kCsrLds;
  uint32_t* lst = fw + 64;
  float* lsd = reinterpret_cast<float*>(fw + 128);
  fw[lane] = lane < deg ? G.g[gb + lane] : DANCE_INV;
  wave_sync();
  const uint32_t grp = lane >> 3, sub = lane & 7u;
  uint4 av[CPL];
  load_row<CPL>(rs, row, true, sub, av);
  const uint32_t* rids = A.rids + s0;
  uint32_t nd = 0, npd = 0, outv;
  uint32_t id[kCsrSlots];
  float d[kCsrSlots];
  uint32_t rem = 0;
#pragma unroll
  for (int e = 0; e < (int)kCsrSlots; ++e) {
    const uint32_t i = (uint32_t)e * 64u + lane;
    uint32_t c = DANCE_INV;
    bool ok = false;
    if (i < deg) {
      c = fw[i];
      ok = true;
    } else if (i < n) {
      c = rids[i - deg];
      ok = c < N && c != row;
      for (uint32_t j = 0; ok && j < deg; ++j) ok = fw[j] != c;
    }
    id[e] = c;
    d[e] = FLT_MAX;
    if (!ok) rem |= 1u << e;
    const uint64_t m = wballot(ok);
    if (m) {
      const uint32_t cnt = popc64(m), pos = mbcnt64(m);
      if (ok) lst[pos] = c;
      wave_sync();
      batch_dist<DT, CPL>(rs, av, lst, lsd, cnt, grp, sub);
      nd += cnt;
      if (ok) d[e] = lsd[pos];
      wave_sync();
    }
  }
  const uint32_t sel = prune_regs<DT, CPL, (int)kCsrSlots>(rs, L, row, R, A.alpha, id, d, rem, lst, lsd, lane, outv, npd);
  if (lane < R) A.gout[gb + lane] = lane < sel ? outv : DANCE_INV;
  if (lane == 0) {
    A.dout[row] = sel;
    if (A.ctr) {
      atomicAdd(ctr_at(A.ctr, kCsrDist), (unsigned long long)nd);
      atomicAdd(ctr_at(A.ctr, kCsrPruneDist), (unsigned long long)npd);
      atomicAdd(ctr_at(A.ctr, kTouchedRows), 1ull);
      atomicAdd(ctr_at(A.ctr, kCsrCandidates), (unsigned long long)nd);
    }
  }
}

// Rows whose candidate list is longer than kCsrRegMax (k_big_sizes gave them
// scratch), with the sort key ~length, so that an ascending sort puts the
// longest lists (the slowest workgroups) first. count[0] counts the rows,
// count[1] those longer than `win` (the prefix of the sorted list that the
// key-window variant of k_csr_long takes).
static __global__ void k_long_rows(uint32_t N, const uint32_t* boff, uint32_t win, uint32_t* list, uint32_t* key,
                                   uint32_t* count) {
  const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= N || boff[row + 1] == boff[row]) return;
  const uint32_t len = boff[row + 1] - boff[row];
  const uint32_t pos = atomicAdd(count, 1u);
  list[pos] = row;
  key[pos] = ~len;
  if (len > win) atomicAdd(count + 1, 1u);
}

// k_csr for one long row per workgroup: the candidate list (same entries as
// k_csr) is distanced by all kLongWaves waves into the row's scratch (bd
// distances, brem removed flags, bmask row-label masks), then
// FilteredRobustPrune runs over it: each selection is the smallest live
// (distance, id, index), reduced over the waves through LDS, and the
// occlusion rule of the selected entry is applied to the live entries.
//
// Selections come in ascending (distance, id, index) order, and an entry's
// fate depends only on the selections made before it, so the list is
// processed in windows of ascending distance keys: the occlusion passes of a
// window cover only its own entries, after replaying on them the selections
// of earlier windows. A row of at most kLongWin entries is one window (the
// whole list); a longer row (label hubs reach 358,549 candidates at c5) takes
// its next window as the ~kLongWin smallest remaining keys (two LDS histogram
// passes: key bits 30..19, then 18..7 inside the crossing bin), kept as an
// index list in LDS, and usually finishes its R selections in the first one.
// kLongWin is the host's CsrArgs::win.
// Entry i belongs to wave (i / 64) % W, lane i % 64 in the distance pass and
// in full-list windows; in a listed window, list slot j belongs to thread j.
// Every pass touches an entry from one thread only. Rows longer than the
// window run with W = kLongWaves; the other long rows (one window each) run
// with fewer waves per workgroup, so that more of them share a CU.
constexpr uint32_t kLongList = 4096;  // LDS capacity of a window list
constexpr uint32_t kLongBins = 4096;  // histogram bins per radix pass

template <int DT, int CPL, int W>
__global__ __launch_bounds__(64 * W) void k_csr_long(RowSet rs, Graph G, Labels L, CsrArgs A, const uint32_t* rows) {
  // W == kLongWaves: rows longer than the key window; fewer waves: the other
  // long rows, which are one window (the whole list), more rows per CU.
  constexpr bool kWin = W == (int)kLongWaves;
  constexpr uint32_t kBlk = 64u * W;
  constexpr uint32_t kBins = kWin ? kLongBins : 1u;
  constexpr uint32_t kList = kWin ? kLongList : 1u;
  __shared__ uint32_t fw[64];
  __shared__ uint32_t wl[W][64];
  __shared__ float wd[W][64];
  __shared__ int rk[W];
  __shared__ uint32_t ri[W], rx[W];
  __shared__ uint32_t out[64], outx[64];
  __shared__ uint32_t hist[kBins];
  __shared__ uint32_t wlist[kList];
  __shared__ uint32_t wtot[W];
  __shared__ uint32_t sh[3];
  const uint32_t row = rows[blockIdx.x];
  const uint32_t w = wave_index(), lane = lane_id();
  const uint32_t tid = w * 64u + lane;
  const uint32_t grp = lane >> 3, sub = lane & 7u;
  const uint32_t N = G.N, R = G.R;
  const size_t gb = (size_t)row * R;
  const uint32_t s0 = A.roff[row], s1 = A.roff[row + 1];
  const uint32_t deg = min(G.d[row], R);
  const uint32_t n = deg + (s1 - s0);
  if (kWin != (n > A.win)) return;  // the other variant's row (uniform)
  if (w == 0) fw[lane] = lane < deg ? G.g[gb + lane] : DANCE_INV;
  __syncthreads();
  const uint32_t base = A.boff[row];
  float* bd = A.bd + base;
  uint8_t* brem = A.brem + base;
  uint32_t* bmask = A.bmask + base;
  const uint32_t* rids = A.rids + s0;
  uint32_t* lst = wl[w];
  float* lsd = wd[w];
  auto id_at = [&](uint32_t i) -> uint32_t { return i < deg ? fw[i] : rids[i - deg]; };
  const bool use_mask = L.off[row + 1] - L.off[row] <= kMaskLabels;
  constexpr uint32_t kStride = kBlk;
  const uint32_t kLongWin = A.win;
  uint32_t nd = 0, npd = 0;
  {
    uint4 av[CPL];
    load_row<CPL>(rs, row, true, sub, av);
    for (uint32_t b = w * 64u; b < n; b += kStride) {
      const uint32_t i = b + lane;
      uint32_t c = DANCE_INV;
      bool ok = false;
      if (i < deg) {
        c = fw[i];
        ok = true;
      } else if (i < n) {
        c = rids[i - deg];
        ok = c < N && c != row;
        for (uint32_t j = 0; ok && j < deg; ++j) ok = fw[j] != c;
      }
      float dist = FLT_MAX;
      const uint64_t m = wballot(ok);
      if (m) {
        const uint32_t cnt = popc64(m), pos = mbcnt64(m);
        if (ok) lst[pos] = c;
        wave_sync();
        batch_dist<DT, CPL>(rs, av, lst, lsd, cnt, grp, sub);
        nd += cnt;
        if (ok) dist = lsd[pos];
        wave_sync();
      }
      if (i < n) {
        brem[i] = ok ? 0 : 1;
        bd[i] = dist;
        bmask[i] = ok && use_mask ? row_mask(L, row, c) : 0u;
      }
    }
  }
  __syncthreads();  // windows read entries of other waves

  // Key of a selectable entry (live, finite distance >= 0): its bit pattern.
  auto key_of = [&](uint32_t i, uint32_t& u) -> bool {
    if (brem[i]) return false;
    const float d = bd[i];
    if (!(d <= FLT_MAX)) return false;
    u = (uint32_t)fkey(d);
    return true;
  };
  // Block-wide exclusive scan of one value per thread; *total gets the sum.
  auto block_scan = [&](uint32_t v, uint32_t* total) -> uint32_t {
    const uint32_t ex = wave_excl_scan_u(v);
    if (lane == 63) wtot[w] = ex + v;
    __syncthreads();
    uint32_t before = 0, all = 0;
    for (uint32_t q = 0; q < (uint32_t)W; ++q) {
      const uint32_t t = wtot[q];
      before += q < w ? t : 0u;
      all += t;
    }
    __syncthreads();  // wtot is rewritten by the next scan
    *total = all;
    return before + ex;
  };
  // Radix pass over the selectable keys >= lo (and with bits 30..19 equal to
  // `bin` unless bin is ~0u): histogram of key bits [shift, shift + 12).
  // Returns the bin where the running count, offset by `prior`, reaches
  // kLongWin (sh[0]) and the count before it (sh[1]); *total as block_scan.
  auto radix_pass = [&](uint32_t lo, uint32_t bin, uint32_t shift, uint32_t prior, uint32_t* total) {
    for (uint32_t q = tid; q < kBins; q += kBlk) hist[q] = 0u;
    __syncthreads();
    for (uint32_t i = tid; i < n; i += kBlk) {
      uint32_t u;
      if (key_of(i, u) && u >= lo && (bin == ~0u || (u >> 19) == bin))
        atomicAdd(&hist[((u >> shift) & 4095u) % kBins], 1u);
    }
    __syncthreads();
    constexpr uint32_t kPer = (kBins + kBlk - 1u) / kBlk;
    uint32_t v = 0;
    for (uint32_t q = 0; q < kPer; ++q) v += tid * kPer + q < kBins ? hist[tid * kPer + q] : 0u;
    const uint32_t ex = prior + block_scan(v, total);
    if (ex < kLongWin && kLongWin <= ex + v) {
      uint32_t c = ex;
      for (uint32_t q = 0; q < kPer; ++q) {
        const uint32_t h = hist[tid * kPer + q];
        if (c + h >= kLongWin) {
          sh[0] = tid * kPer + q;
          sh[1] = c;
          break;
        }
        c += h;
      }
    }
    __syncthreads();
  };

  uint32_t sel = 0;
  uint32_t lo = 0u, hi = ~0u;
  bool listed = false;
  uint32_t m = n;  // entries of the current window's iteration space
  bool done = false;
  bool first = true;
  while (!done) {
    if (!first && hi == ~0u) break;  // the last window is done
    if (kWin && (!first || n > kLongWin)) {
      if (!first) lo = hi + 1u;
      uint32_t total;
      radix_pass(lo, ~0u, 19u, 0u, &total);
      if (total == 0u) break;
      if (total <= kLongWin) {
        hi = ~0u;
      } else {
        const uint32_t bin = sh[0], prior = sh[1];
        __syncthreads();
        uint32_t t2;
        radix_pass(lo, bin, 7u, prior, &t2);
        hi = (bin << 19) | (sh[0] << 7) | 127u;
        __syncthreads();
      }
      if (tid == 0) sh[2] = 0u;
      __syncthreads();
      for (uint32_t i = tid; i < n; i += kBlk) {
        uint32_t u;
        if (key_of(i, u) && u >= lo && u <= hi) {
          const uint32_t p = atomicAdd(&sh[2], 1u);
          if (p < kList) wlist[p] = i;
        }
      }
      __syncthreads();
      const uint32_t cnt = sh[2];
      listed = cnt <= kList;
      m = listed ? cnt : n;
      __syncthreads();
    }
    first = false;
    // Entry of iteration slot j of the window (j < m), or none.
    auto entry = [&](uint32_t j, uint32_t& i) -> bool {
      if (j >= m) return false;
      if (listed) {
        i = wlist[j % kList];  // j < m <= kList when listed
        return true;
      }
      i = j;
      if (lo == 0u && hi == ~0u) return true;
      uint32_t u;
      return key_of(i, u) && u >= lo && u <= hi;
    };
    // Each lane tracks the smallest live (distance, id) of its own window
    // entries and the iteration slot that holds it (live ids are unique, so
    // the slot only names the entry's owner).
    int bk = INT_MAX;
    uint32_t bid = DANCE_INV, bix = DANCE_INV;
    auto consider = [&](float d, uint32_t c, uint32_t j) {
      if (!(d <= FLT_MAX)) return;
      const int k = fkey(d);
      if (k < bk || (k == bk && c < bid)) {
        bk = k;
        bid = c;
        bix = j;
      }
    };
    // The occlusion rule of selection (gi, gx) on the window's live entries;
    // with track, the survivors' minimum for the next selection.
    auto occlude = [&](uint32_t gi, uint32_t gx, bool track) {
      const uint32_t msel = use_mask ? bmask[gx] : 0u;
      uint4 bv[CPL];
      load_row<CPL>(rs, gi, true, sub, bv);
      for (uint32_t jb = w * 64u; jb < m; jb += kStride) {
        uint32_t i = 0;
        bool live = entry(jb + lane, i) && i != gx && !brem[i];
        const uint32_t c = live ? id_at(i) : DANCE_INV;
        const bool need = live && (use_mask ? (bmask[i] & ~msel) == 0u : covers(L, row, gi, c));
        const uint64_t mk = wballot(need);
        if (mk) {
          const uint32_t cnt = popc64(mk), pos = mbcnt64(mk);
          if (need) lst[pos] = c;
          wave_sync();
          batch_dist<DT, CPL>(rs, bv, lst, lsd, cnt, grp, sub);
          npd += cnt;
          if (need) {
            const float pd = lsd[pos];
            if (pd > 0.0f && A.alpha * pd <= bd[i]) {
              brem[i] = 1;
              live = false;
            }
          }
          wave_sync();
        }
        if (track && live) consider(bd[i], c, jb + lane);
      }
    };
    // earlier windows' selections, then the window's own minimum
    for (uint32_t q = 0; q < sel; ++q) occlude(out[q], outx[q], q + 1 == sel);
    if (sel == 0) {
      for (uint32_t jb = w * 64u; jb < m; jb += kStride) {
        uint32_t i = 0;
        if (entry(jb + lane, i) && !brem[i]) consider(bd[i], id_at(i), jb + lane);
      }
    }
    while (true) {
      const int M = wave_min_i(bk);
      const uint32_t I = wave_min_u(bk == M ? bid : DANCE_INV);
      const uint32_t X = wave_min_u(bk == M && bid == I ? bix : DANCE_INV);
      if (lane == 0) {
        rk[w] = M;
        ri[w] = I;
        rx[w] = X;
      }
      __syncthreads();
      const int mk = lane < (uint32_t)W ? rk[lane] : INT_MAX;
      const uint32_t mi = lane < (uint32_t)W ? ri[lane] : DANCE_INV;
      const uint32_t mx = lane < (uint32_t)W ? rx[lane] : DANCE_INV;
      __syncthreads();  // rk / ri / rx are rewritten by the next selection
      const int GM = wave_min_i(mk);
      if (GM == INT_MAX) break;  // window exhausted
      const uint32_t GI = wave_min_u(mk == GM ? mi : DANCE_INV);
      const uint32_t GJ = wave_min_u(mk == GM && mi == GI ? mx : DANCE_INV);
      const uint32_t GX = listed ? wlist[GJ % kList] : GJ;
      if (tid == 0) {
        out[sel] = GI;
        outx[sel] = GX;
      }
      if (tid == GJ % kBlk) brem[GX] = 1;  // the slot's owner, which alone reads it in this window
      if (++sel == R) {  // removals after the last selection change nothing
        done = true;
        break;
      }
      bk = INT_MAX;
      bid = bix = DANCE_INV;
      occlude(GI, GX, true);
    }
    __syncthreads();  // out / outx / brem visible to the next window
  }
  __syncthreads();
  if (w == 0) {
    if (lane < R) A.gout[gb + lane] = lane < sel ? out[lane] : DANCE_INV;
    if (lane == 0) A.dout[row] = sel;
  }
  if (A.ctr && lane == 0) {
    atomicAdd(ctr_at(A.ctr, kCsrDist), (unsigned long long)nd);
    atomicAdd(ctr_at(A.ctr, kCsrPruneDist), (unsigned long long)npd);
    atomicAdd(ctr_at(A.ctr, kCsrCandidates), (unsigned long long)nd);
    if (w == 0) {
      atomicAdd(ctr_at(A.ctr, kTouchedRows), 1ull);
      atomicAdd(ctr_at(A.ctr, kBigRows), 1ull);
      atomicMax(ctr_at(A.ctr, kBigMax), (unsigned long long)n);
    }
  }
}

// ---------------------------------------------------------------------------
// Publish step for a published degree PR below the build degree
// (gpu_vamana_filtered.cu:6328-6432).
// ---------------------------------------------------------------------------
constexpr uint32_t kPubLocal = kCsrRegMax;  // candidate lists up to this length stay in LDS
// LDS words per wave of k_publish: forward row, one distance batch, then the
// local candidate ids, distances and state bytes.
constexpr uint32_t kPubLds = 64u + 128u + 2u * kPubLocal + kPubLocal / 4u;

// canonical_rare_label_shortlist_warp (gpu_vamana_filtered.cu:5285-5406)
// over n candidates (cid, cd) with state bytes cst; entry i belongs to lane
// i % 64, which alone reads and writes cst[i]. For each row label that is not
// universal, is below num_labels and has at most PR*PR points: up to quota =
// max(1, PR / |labels(row)|) picks of the smallest (distance, id, position)
// carrier not yet picked for that label, each output unless an earlier label
// already output it. Then the smallest candidates not yet output fill up to
// PR. Only ids != DANCE_INV with distance <= FLT_MAX are picked. Lane k <
// count receives the k-th output. State bits: 1 output, 2 picked for the
// current label, 4 carries the current label.
__device__ uint32_t rare_shortlist(const Labels& L, uint32_t N, uint32_t row, uint32_t PR, uint32_t n,
                                   const uint32_t* cid, const float* cd, uint8_t* cst, uint32_t lane, uint32_t& oid,
                                   float& od) {
  // smallest pickable (distance, id, position) with (state & mask) == want;
  // returns its position (DANCE_INV: none), id and distance
  auto pick = [&](uint32_t mask, uint32_t want, uint32_t& I, float& D) -> uint32_t {
    int bk = INT_MAX;
    uint32_t bid = DANCE_INV, bpos = DANCE_INV;
    for (uint32_t i = lane; i < n; i += 64) {
      if ((cst[i] & mask) != want) continue;
      const uint32_t c = cid[i];
      const float d = cd[i];
      if (c == DANCE_INV || !(d <= FLT_MAX)) continue;
      const int k = fkey(d);
      if (k < bk || (k == bk && c < bid)) {  // positions ascend per lane: ties keep the first
        bk = k;
        bid = c;
        bpos = i;
      }
    }
    const int M = wave_min_i(bk);
    if (M == INT_MAX) return DANCE_INV;
    I = wave_min_u(bk == M ? bid : DANCE_INV);
    D = __int_as_float(M);
    return wave_min_u(bk == M && bid == I ? bpos : DANCE_INV);
  };
  for (uint32_t i = lane; i < n; i += 64) cst[i] = 0;
  uint32_t count = 0;
  oid = DANCE_INV;
  od = FLT_MAX;
  const uint32_t l0 = L.off[row], l1 = L.off[row + 1], nl = l1 - l0;
  const uint32_t quota = nl ? max(1u, PR / nl) : 0u;
  const uint64_t risk = (uint64_t)PR * PR;
  for (uint32_t lp = l0; lp < l1 && count < PR; ++lp) {
    const uint32_t label = L.lab[lp];
    if (label == L.universal || label >= L.num_labels || (uint64_t)(L.lpo[label + 1] - L.lpo[label]) > risk) continue;
    for (uint32_t i = lane; i < n; i += 64) {
      const uint32_t c = cid[i];
      const bool car = c < N && has_exact(L, c, label);
      cst[i] = (uint8_t)((cst[i] & 1u) | (car ? 4u : 0u));
    }
    for (uint32_t k = 0; k < quota && count < PR; ++k) {
      uint32_t I;
      float D;
      const uint32_t X = pick(6u, 4u, I, D);
      if (X == DANCE_INV) break;
      uint32_t was = 0;
      if (lane == (X & 63u)) {
        was = cst[X] & 1u;
        cst[X] |= 3u;
      }
      if (!rdlane_u(was, (int)(X & 63u))) {
        if (lane == count) {
          oid = I;
          od = D;
        }
        ++count;
      }
    }
  }
  while (count < PR) {
    uint32_t I;
    float D;
    const uint32_t X = pick(1u, 0u, I, D);
    if (X == DANCE_INV) break;
    if (lane == (X & 63u)) cst[X] |= 1u;
    if (lane == count) {
      oid = I;
      od = D;
    }
    ++count;
  }
  return count;
}

struct PubArgs {
  float alpha;
  uint32_t PR;
  const uint32_t* roff;  // reverse pass: N+1 reverse offsets of the forward pass's graph
  const uint32_t* rids;  // reverse pass: reverse sources
  const uint32_t* boff;  // reverse pass: N+1 scratch offsets of lists longer than kPubLocal
  uint32_t* bid;
  float* bd;
  uint8_t* bst;
  uint32_t* gout;  // N x PR
  uint32_t* dout;  // N
  unsigned long long* ctr;
};

// One row of the publish step, one wave per row.
// Forward pass (REV = false; canonical_fixed_rare_shortlist :5408-5431 +
// canonical_exact_prune): candidates are the row of G (build degree R <= 64),
// distanced, shortlisted to PR and pruned to PR into gout.
// Reverse pass (REV = true; canonical_reverse_candidate_count/fill,
// canonical_csr_candidate_distances, canonical_csr_rare_shortlist
// :5036-5106, :5433-5450 + canonical_exact_prune): rows with reverse sources
// in the forward pass's graph G (stride PR) take their forward row followed by
// the sources not in it (not the row itself), every distance recomputed, and
// are shortlisted and pruned again, in place (gout == G.g: each wave reads
// only its own row, before writing it). Rows without sources keep their row.
// Sources that duplicate the forward row stay in the list as DANCE_INV
// entries, never picked: the relative order of the others, which alone
// breaks ties, is that of the reference's compacted list.
template <int DT, int CPL, bool REV>
__global__ __launch_bounds__(kBlock) void k_publish(RowSet rs, Graph G, Labels L, PubArgs A) {
  extern __shared__ uint32_t smem[];
  const uint32_t w = wave_index();
  const uint32_t row = xcd_block(grid_block(), grid_blocks()) * kWaves + w;
  const uint32_t N = G.N;
  if (row >= N) return;
  const uint32_t lane = lane_id();
  uint32_t s0 = 0, s1 = 0;
  if constexpr (REV) {
    s0 = A.roff[row];
    s1 = A.roff[row + 1];
    if (s0 == s1) return;
  }
  uint32_t* fw = smem + w * kPubLds;
  uint32_t* lst = fw + 64;
  float* lsd = reinterpret_cast<float*>(fw + 128);
  uint32_t* cid = fw + 192;
  float* cdist = reinterpret_cast<float*>(cid + kPubLocal);
  uint8_t* cst = reinterpret_cast<uint8_t*>(cid + 2u * kPubLocal);
  const uint32_t deg = min(G.d[row], G.R);  // G.R <= 64
  fw[lane] = lane < deg ? G.g[(size_t)row * G.R + lane] : DANCE_INV;
  wave_sync();
  const uint32_t n = deg + (s1 - s0);
  if (n > kPubLocal) {  // reverse pass only: deg <= 64
    const uint32_t b = A.boff[row];
    cid = A.bid + b;
    cdist = A.bd + b;
    cst = A.bst + b;
  }
  const uint32_t grp = lane >> 3, sub = lane & 7u;
  uint4 av[CPL];
  load_row<CPL>(rs, row, true, sub, av);
  uint32_t nd = 0;
  for (uint32_t b = 0; b < n; b += 64) {
    const uint32_t i = b + lane;
    uint32_t c = DANCE_INV;
    if (i < deg) {
      c = fw[i];
    } else if (i < n) {
      c = A.rids[s0 + (i - deg)];
      bool dup = c >= N || c == row;
      for (uint32_t j = 0; !dup && j < deg; ++j) dup = fw[j] == c;
      if (dup) c = DANCE_INV;
    }
    const bool ok = i < n && c < N;  // ids outside the graph get no distance and are never picked
    float dist = __builtin_inff();
    const uint64_t m = wballot(ok);
    if (m) {
      const uint32_t cnt = popc64(m), pos = mbcnt64(m);
      if (ok) lst[pos] = c;
      wave_sync();
      batch_dist<DT, CPL>(rs, av, lst, lsd, cnt, grp, sub);
      nd += cnt;
      if (ok) dist = lsd[pos];
      wave_sync();
    }
    if (i < n) {
      cid[i] = c;
      cdist[i] = dist;
    }
  }
  uint32_t oid;
  float od;
  const uint32_t cnt = rare_shortlist(L, N, row, A.PR, n, cid, cdist, cst, lane, oid, od);
  const uint32_t id1[1] = {oid};
  const float d1[1] = {od};
  uint32_t outv, npd = 0;
  const uint32_t sel =
      prune_regs<DT, CPL, 1>(rs, L, row, A.PR, A.alpha, id1, d1, lane < cnt ? 0u : 1u, lst, lsd, lane, outv, npd);
  if (lane < A.PR) A.gout[(size_t)row * A.PR + lane] = lane < sel ? outv : DANCE_INV;
  if (lane == 0) {
    A.dout[row] = sel;
    if (A.ctr) {
      atomicAdd(ctr_at(A.ctr, kPubDist), (unsigned long long)(nd + npd));
      if (REV) atomicAdd(ctr_at(A.ctr, kPubTouched), 1ull);
    }
  }
}

// filtered_graph_diagnostics_kernel (gpu_vamana_filtered.cu:2716-2774).
// u32 slots: invalid, self, low_common, deg_min, deg_max, common_min,
// common_max; u64 slots: out_edges, common_edges, label_checks,
// label_rejects, universal_passes.
static __global__ void k_diagnostics(Graph G, Labels L, uint32_t* d32, unsigned long long* d64) {
  const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
  const bool in = row < G.N;
  const uint32_t deg = in ? G.d[row] : 0u;
  uint32_t invalid = 0, self = 0, common = 0, checks = 0, uni = 0;
  const uint32_t n = in ? min(deg, G.R) : 0u;
  for (uint32_t j = 0; j < n; ++j) {
    const uint32_t nb = G.g[(size_t)row * G.R + j];
    if (nb >= G.N) {
      ++invalid;
      continue;
    }
    if (nb == row) {
      ++self;
      continue;
    }
    ++checks;
    // has_common with the universal rule, noting universal passes
    uint32_t i = L.off[row], k = L.off[nb];
    const uint32_t ie = L.off[row + 1], ke = L.off[nb + 1];
    while (i < ie && k < ke) {
      const uint32_t x = L.lab[i], y = L.lab[k];
      if (x == L.universal || y == L.universal) {
        ++uni;
        ++common;
        break;
      }
      if (x == y) {
        ++common;
        break;
      }
      if (x < y)
        ++i;
      else
        ++k;
    }
  }
  // one atomic per wave and counter (wave sums fit in 32 bits: <= 64 * R)
  auto add = [](int a, int b) { return a + b; };
  const uint32_t s_invalid = (uint32_t)wave_reduce_i((int)invalid, 0, add);
  const uint32_t s_self = (uint32_t)wave_reduce_i((int)self, 0, add);
  const uint32_t s_low = (uint32_t)wave_reduce_i(in && common < 2 ? 1 : 0, 0, add);
  const uint32_t s_deg = (uint32_t)wave_reduce_i((int)deg, 0, add);
  const uint32_t s_common = (uint32_t)wave_reduce_i((int)common, 0, add);
  const uint32_t s_checks = (uint32_t)wave_reduce_i((int)checks, 0, add);
  const uint32_t s_uni = (uint32_t)wave_reduce_i((int)uni, 0, add);
  const uint32_t mn_deg = wave_min_u(in ? deg : 0xFFFFFFFFu), mx_deg = wave_max_u(deg);
  const uint32_t mn_com = wave_min_u(in ? common : 0xFFFFFFFFu), mx_com = wave_max_u(common);
  const bool any_row = wballot(in) != 0ull;
  if (lane_id() == 0 && any_row) {
    if (s_invalid) atomicAdd(d32 + 0, s_invalid);
    if (s_self) atomicAdd(d32 + 1, s_self);
    if (s_low) atomicAdd(d32 + 2, s_low);
    atomicMin(d32 + 3, mn_deg);
    atomicMax(d32 + 4, mx_deg);
    atomicMin(d32 + 5, mn_com);
    atomicMax(d32 + 6, mx_com);
    atomicAdd(d64 + 0, (unsigned long long)s_deg);
    atomicAdd(d64 + 1, (unsigned long long)s_common);
    atomicAdd(d64 + 2, (unsigned long long)s_checks);
    atomicAdd(d64 + 3, (unsigned long long)(s_checks - s_common));
    if (s_uni) atomicAdd(d64 + 4, (unsigned long long)s_uni);
  }
}

// Per-round counts of the round line (gpu_vamana_filtered.cu:6106-6297), one
// wave per row: out[0] += rows whose new row differs from the round's input
// row (degree differs, or a new entry is absent from the old row: the test of
// canonical_exact_prune / canonical_exact_prune_csr, :4979-4990, :5218-5228);
// out[1] += rows with at least one reverse source (the touched flag of
// canonical_reverse_candidate_count, :5049).
static __global__ void k_round_changes(uint32_t N, uint32_t R, const uint32_t* old_g, const uint32_t* old_d,
                                       const uint32_t* new_g, const uint32_t* new_d, const uint32_t* roff,
                                       unsigned long long* out) {
  const uint32_t row = blockIdx.x * (blockDim.x / 64) + wave_index(), lane = lane_id();
  if (row >= N) return;
  const uint32_t od = min(old_d[row], R), nd = min(new_d[row], R);
  bool changed = od != nd;
  for (uint32_t b = 0; !changed && b < nd; b += 64) {
    const uint32_t j = b + lane;
    const uint32_t v = j < nd ? new_g[(size_t)row * R + j] : DANCE_INV;
    bool found = j >= nd;
    for (uint32_t k = 0; k < od; ++k) found |= old_g[(size_t)row * R + k] == v;
    changed = wballot(!found) != 0ull;
  }
  if (lane == 0) {
    if (changed) atomicAdd(out, 1ull);
    if (roff[row + 1] > roff[row]) atomicAdd(out + 1, 1ull);
  }
}

// Per-row figures of canonical_print_round_diagnostics (:94-160), one thread
// per row over the first min(degree, R) entries: compat[row] = entries whose
// id is < N and that carry one of the row's labels (any entry when the row
// has the universal label); minpl[row] = the least, over the row's labels
// other than the universal one, of the entries carrying that label (compat
// when the row has no such label).
static __global__ void k_degree_profile(Graph G, Labels L, uint32_t* compat, uint32_t* minpl) {
  const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= G.N) return;
  const uint32_t n = min(G.d[row], G.R);
  const uint32_t* nb = G.g + (size_t)row * G.R;
  const uint32_t b = L.off[row], e = L.off[row + 1];
  uint32_t mn = G.R, c = 0;
  bool specific = false;
  for (uint32_t p = b; p < e; ++p) {
    const uint32_t l = L.lab[p];
    if (l == L.universal) continue;
    specific = true;
    uint32_t k = 0;
    for (uint32_t i = 0; i < n; ++i) k += nb[i] < G.N && has_exact(L, nb[i], l);
    mn = min(mn, k);
  }
  for (uint32_t i = 0; i < n; ++i) {
    const uint32_t v = nb[i];
    bool shares = false;
    for (uint32_t p = b; !shares && p < e && v < G.N; ++p)
      shares = L.lab[p] == L.universal || has_exact(L, v, L.lab[p]);
    c += shares;
  }
  compat[row] = c;
  minpl[row] = specific ? mn : c;
}

}  // namespace filt
}  // namespace dance
