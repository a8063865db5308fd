// CPU oracle of the GPU-FilteredVamana "canonical_v2" build.
//
// TEST INFRASTRUCTURE ONLY (see vamana_oracle.cpp). A sequential restatement
// of /root/reference/src/gpu_vamana_filtered.cu's release path:
//   gpu_vamana_filtered_build_impl (:6511-7067) -> deterministic random
//   backbone (:716-744, seed 42, degree min(16, R)) -> canonical rounds
//   (canonical_round0_from_host_backbone_typed, :5663-6483) -> diagnostics
//   (filtered_graph_diagnostics_kernel, :2716-2774).
// Float input is searched on fp16 rows (:6497-6503); the distance is the
// canonical one of vamana_oracle.cpp (binary16 differences and squares,
// filtered.cu:4036-4047).
// The reference fills its reverse CSR with atomics, but the CSR prune selects
// by (distance, id) over unique ids, so its result does not depend on that
// order; this oracle uses ascending sources.

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>
#include <omp.h>

extern "C" float oracle_distance(const void* data, int dtype, uint32_t dim, uint32_t a, uint32_t b);

namespace {

constexpr uint32_t INV = 0xFFFFFFFFu;

struct Ctx {
  const void* data;
  int dtype;
  uint32_t N, dim, R;
  const uint32_t* off;     // N+1
  const uint32_t* lab;     // sorted unique per row
  uint32_t num_labels;
  uint32_t universal;
  const uint32_t* starts;  // num_labels
  std::vector<uint32_t> lpo, lpts;  // label -> points CSR (ascending rows)
  float D(uint32_t a, uint32_t b) const { return oracle_distance(data, dtype, dim, a, b); }
};

inline uint32_t fhash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// point_has_exact_label_device (:557-573)
bool has_exact(const Ctx& c, uint32_t p, uint32_t label) {
  for (uint32_t i = c.off[p]; i < c.off[p + 1]; ++i) {
    if (c.lab[i] == label) return true;
    if (c.lab[i] > label) break;
  }
  return false;
}

// has_common_label_device (:495-528)
bool has_common(const Ctx& c, uint32_t a, uint32_t b, uint32_t universal) {
  uint32_t i = c.off[a], ie = c.off[a + 1], j = c.off[b], je = c.off[b + 1];
  while (i < ie && j < je) {
    uint32_t x = c.lab[i], y = c.lab[j];
    if (x == universal || y == universal) return true;
    if (x == y) return true;
    if (x < y) ++i; else ++j;
  }
  return false;
}

// filtered_selected_covers_common_labels (include/filtered_label_coverage.cuh:7-44)
bool covers(const Ctx& c, uint32_t target, uint32_t selected, uint32_t cand) {
  uint32_t ti = c.off[target], te = c.off[target + 1], ci = c.off[cand], ce = c.off[cand + 1];
  const uint32_t sb = c.off[selected], se = c.off[selected + 1];
  while (ti < te && ci < ce) {
    uint32_t tl = c.lab[ti], cl = c.lab[ci];
    if (tl < cl) ++ti;
    else if (cl < tl) ++ci;
    else {
      bool found = false;
      for (uint32_t s = sb; s < se; ++s) {
        if (c.lab[s] == tl) { found = true; break; }
        if (c.lab[s] > tl) break;
      }
      if (!found) return false;
      ++ti;
      ++ci;
    }
  }
  return true;
}

// Canonical pool (:4156-4263): no early reject; worst by (distance, id);
// selection of the unexpanded minimum by (distance, id).
struct CPool {
  uint32_t cap, count = 0;
  std::vector<uint32_t> ids;
  std::vector<float> d;
  std::vector<uint8_t> ex;
  int worst_pos = -1;
  float worst_d = -FLT_MAX;
  explicit CPool(uint32_t c) : cap(c), ids(c, INV), d(c, FLT_MAX), ex(c, 0) {}
  void recompute_worst() {
    float ld = -FLT_MAX;
    uint32_t lid = 0;
    int lp = -1;
    for (uint32_t p = 0; p < count; ++p)
      if (d[p] > ld || (d[p] == ld && ids[p] > lid)) { ld = d[p]; lid = ids[p]; lp = (int)p; }
    worst_pos = lp;
    worst_d = ld;
  }
  void insert(uint32_t id, float dist) {
    if (id == INV) return;
    int dup = -1;
    for (uint32_t p = 0; p < count; ++p)
      if (ids[p] == id) { dup = (int)p; break; }
    bool changed = false;
    if (dup >= 0) {
      if (dist < d[dup]) { d[dup] = dist; ex[dup] = 0; changed = true; }
    } else if (count < cap) {
      ids[count] = id; d[count] = dist; ex[count] = 0; ++count; changed = true;
    } else {
      recompute_worst();
      const uint32_t wid = worst_pos >= 0 ? ids[worst_pos] : 0;
      if (worst_pos >= 0 && (dist < worst_d || (dist == worst_d && id < wid))) {
        ids[worst_pos] = id; d[worst_pos] = dist; ex[worst_pos] = 0; changed = true;
      }
    }
    if (changed) recompute_worst();
  }
  int select() const {
    float bd = FLT_MAX;
    uint32_t bid = 0xFFFFFFFFu;
    int bp = -1;
    for (uint32_t p = 0; p < count; ++p)
      if (!ex[p] && (d[p] < bd || (d[p] == bd && ids[p] < bid))) { bd = d[p]; bid = ids[p]; bp = (int)p; }
    return bp;
  }
};

// canonical_filtered_task_search (:4265-4426), retain_posting_anchor = 0.
void task_search(const Ctx& c, const uint32_t* ga, const uint32_t* da, uint32_t row, uint32_t label,
                 uint32_t pool_cap, uint32_t keep, uint32_t steps, uint32_t* out_ids, float* out_d) {
  for (uint32_t i = 0; i < keep; ++i) { out_ids[i] = INV; out_d[i] = FLT_MAX; }
  const uint32_t N = c.N, R = c.R;
  if (row >= N || label >= c.num_labels || label == c.universal) return;
  CPool P(pool_cap);
  const uint32_t start = c.starts[label];
  if (start < N && start != row) P.insert(start, c.D(row, start));
  {
    const uint32_t pb = c.lpo[label], pc = c.lpo[label + 1] - pb;
    const uint32_t seeds = std::min(std::min(16u, 16u), pc);
    for (uint32_t s = 0; s < seeds; ++s) {
      const uint32_t seed = c.lpts[pb + (fhash(row + s * 7919u + label * 17u) % pc)];
      if (seed >= N || seed == row) continue;
      P.insert(seed, c.D(row, seed));
    }
  }
  const uint32_t deg = std::min(da[row], R);
  for (uint32_t j = 0; j < deg; ++j) {
    const uint32_t cand = ga[(size_t)row * R + j];
    if (cand >= N || cand == row || !has_exact(c, cand, label)) continue;
    P.insert(cand, c.D(row, cand));
  }
  for (uint32_t step = 0; step < steps; ++step) {
    const int pos = P.select();
    if (pos < 0) break;
    P.ex[pos] = 1;
    const uint32_t e = P.ids[pos];
    const uint32_t de = std::min(da[e], R);
    for (uint32_t j = 0; j < de; ++j) {
      const uint32_t cand = ga[(size_t)e * R + j];
      if (cand >= N || cand == row || !has_exact(c, cand, label)) continue;
      P.insert(cand, c.D(row, cand));
    }
  }
  for (uint32_t i = 0; i < keep && i < P.count; ++i) { out_ids[i] = P.ids[i]; out_d[i] = P.d[i]; }
}

// canonical_ordinary_search (:4529-4670), restricted traversal, all slots out.
void ordinary_search(const Ctx& c, const uint32_t* ga, const uint32_t* da, uint32_t row, uint32_t pool_cap,
                     uint32_t keep, uint32_t steps, uint32_t global_start, uint32_t* out_ids, float* out_d) {
  const uint32_t N = c.N, R = c.R;
  CPool P(pool_cap);
  auto compatible = [&](uint32_t cand) {
    for (uint32_t p = c.off[row]; p < c.off[row + 1]; ++p)
      if (has_exact(c, cand, c.lab[p])) return true;
    return false;
  };
  for (uint32_t p = c.off[row]; p < c.off[row + 1]; ++p) {
    const uint32_t label = c.lab[p];
    if (label >= c.num_labels) continue;
    const uint32_t start = c.starts[label];
    if (start < N && start != row) P.insert(start, c.D(row, start));
    const uint32_t pb = c.lpo[label], pc = c.lpo[label + 1] - pb;
    const uint32_t seeds = std::min(64u, pc);
    for (uint32_t s = 0; s < seeds; ++s) {
      const uint32_t seed = c.lpts[pb + (fhash(row + s * 7919u + label * 17u) % pc)];
      if (seed >= N || seed == row) continue;
      P.insert(seed, c.D(row, seed));
    }
  }
  if (global_start < N && global_start != row && compatible(global_start))
    P.insert(global_start, c.D(row, global_start));
  const uint32_t deg = std::min(da[row], R);
  for (uint32_t j = 0; j < deg; ++j) {
    const uint32_t cand = ga[(size_t)row * R + j];
    if (cand >= N || cand == row || !compatible(cand)) continue;
    P.insert(cand, c.D(row, cand));
  }
  for (uint32_t step = 0; step < steps; ++step) {
    const int pos = P.select();
    if (pos < 0) break;
    P.ex[pos] = 1;
    const uint32_t e = P.ids[pos];
    const uint32_t de = std::min(da[e], R);
    for (uint32_t j = 0; j < de; ++j) {
      const uint32_t cand = ga[(size_t)e * R + j];
      if (cand >= N || cand == row || !compatible(cand)) continue;
      P.insert(cand, c.D(row, cand));
    }
  }
  for (uint32_t i = 0; i < keep; ++i) {
    out_ids[i] = i < P.count ? P.ids[i] : INV;
    out_d[i] = i < P.count ? P.d[i] : FLT_MAX;
  }
}

// canonical_merge_one_warp (:4672-4701)
void merge_one(uint32_t cand, float dist, uint32_t row, uint32_t N, uint32_t C, uint32_t* w, float* wd,
               uint32_t& count) {
  if (cand >= N || cand == row || count >= C) return;
  for (uint32_t p = 0; p < count; ++p)
    if (w[p] == cand) {
      if (dist < wd[p]) wd[p] = dist;
      return;
    }
  w[count] = cand;
  wd[count] = dist;
  ++count;
}

// canonical_merge_candidates (:4703-4842) with label-quota compaction;
// bridges and posting anchors are off on the release path.
uint32_t merge_row(const Ctx& c, const uint32_t* ga, const uint32_t* da, uint32_t row, uint32_t C,
                   uint32_t per_label_keep, uint32_t ordinary_keep, const uint32_t* task_ids, const float* task_d,
                   uint32_t* w, float* wd) {
  const uint32_t N = c.N, R = c.R;
  std::vector<uint32_t> oid(w, w + ordinary_keep);
  std::vector<float> od(wd, wd + ordinary_keep);
  for (uint32_t i = 0; i < C; ++i) { w[i] = INV; wd[i] = FLT_MAX; }
  uint32_t count = 0;
  for (uint32_t p = c.off[row]; p < c.off[row + 1]; ++p)
    for (uint32_t i = 0; i < per_label_keep; ++i)
      merge_one(task_ids[(size_t)p * per_label_keep + i], task_d[(size_t)p * per_label_keep + i], row, N, C, w, wd,
                count);
  const uint32_t deg = std::min(da[row], R);
  for (uint32_t i = 0; i < deg; ++i) {
    const uint32_t cand = ga[(size_t)row * R + i];
    if (cand < N && cand != row && has_common(c, row, cand, 0xFFFFFFFFu)) merge_one(cand, FLT_MAX, row, N, C, w, wd, count);
  }
  for (uint32_t i = 0; i < ordinary_keep; ++i) merge_one(oid[i], od[i], row, N, C, w, wd, count);
  const uint32_t lc = c.off[row + 1] - c.off[row];
  if (lc > 0 && lc <= 16) {
    uint32_t assigned[16] = {};
    uint32_t quota = (R + lc - 1) / lc;
    if (quota < per_label_keep) quota = per_label_keep;
    uint32_t balanced = 0;
    for (uint32_t i = 0; i < count; ++i) {
      const uint32_t cand = w[i];
      uint32_t bq = 0xFFFFFFFFu, bcard = 0xFFFFFFFFu;
      for (uint32_t q = 0; q < lc; ++q) {
        const uint32_t label = c.lab[c.off[row] + q];
        if (assigned[q] >= quota || !has_exact(c, cand, label)) continue;
        // labels >= num_labels have no posting list: cardinality 0 (the
        // reference indexes past its offsets array there)
        const uint32_t card = label < c.num_labels ? c.lpo[label + 1] - c.lpo[label] : 0u;
        if (bq == 0xFFFFFFFFu || card < bcard || (card == bcard && label < c.lab[c.off[row] + bq])) {
          bq = q;
          bcard = card;
        }
      }
      if (bq == 0xFFFFFFFFu) continue;
      if (balanced != i) { w[balanced] = cand; wd[balanced] = wd[i]; }
      ++assigned[bq];
      ++balanced;
    }
    count = balanced;
  }
  return count;
}

// canonical_exact_prune / canonical_exact_prune_csr (:4876-4994, :5130-5230):
// FilteredRobustPrune, selection by (distance, id, position).
uint32_t filtered_prune(const Ctx& c, uint32_t row, const uint32_t* ids, const float* ds, uint32_t n, float alpha,
                        uint32_t* out, uint32_t R) {
  std::vector<uint8_t> removed(n, 0);
  uint32_t sel = 0;
  for (uint32_t i = 0; i < R; ++i) out[i] = INV;
  while (sel < R) {
    float bd = FLT_MAX;
    uint32_t bid = 0xFFFFFFFFu, bi = 0xFFFFFFFFu;
    for (uint32_t i = 0; i < n; ++i) {
      if (removed[i]) continue;
      if (ds[i] < bd || (ds[i] == bd && (ids[i] < bid || (ids[i] == bid && i < bi)))) { bd = ds[i]; bid = ids[i]; bi = i; }
    }
    if (bi == 0xFFFFFFFFu) break;
    out[sel++] = bid;
    removed[bi] = 1;
    for (uint32_t i = 0; i < n; ++i) {
      if (removed[i]) continue;
      if (!covers(c, row, bid, ids[i])) continue;
      const float pd = c.D(bid, ids[i]);
      if (pd > 0.0f && alpha * pd <= ds[i]) removed[i] = 1;
    }
  }
  return sel;
}

// canonical_rare_label_shortlist_warp (:5291-5406): keeps at most R of the
// n candidates. For each row label (CSR order) that is not universal, is
// below num_labels and has at most R*R points, up to quota = max(1, R / |F_row|)
// picks of the smallest (distance, id, position) carrying the label, each
// pick output unless an earlier label already output it; then the smallest
// remaining candidates fill up to R. Only ids != INV with distance <=
// FLT_MAX are picked.
uint32_t rare_shortlist(const Ctx& c, uint32_t row, uint32_t R, const uint32_t* ids, const float* ds, uint32_t n,
                        uint32_t* out_ids, float* out_ds) {
  std::vector<uint8_t> state(n, 0);  // bit 1: output, bit 2: picked for the current label
  uint32_t count = 0;
  const uint32_t nl = c.off[row + 1] - c.off[row];
  const uint32_t quota = nl ? std::max(1u, R / nl) : 0u;
  const uint64_t risk = (uint64_t)R * R;
  auto better = [&](uint32_t i, uint32_t best) {
    if (best == INV) return true;
    return ds[i] < ds[best] || (ds[i] == ds[best] && (ids[i] < ids[best] || (ids[i] == ids[best] && i < best)));
  };
  auto pickable = [&](uint32_t i) { return ids[i] != INV && ds[i] <= FLT_MAX; };
  for (uint32_t lp = c.off[row]; lp < c.off[row + 1] && count < R; ++lp) {
    const uint32_t label = c.lab[lp];
    if (label == c.universal || label >= c.num_labels || (uint64_t)(c.lpo[label + 1] - c.lpo[label]) > risk) continue;
    for (uint32_t i = 0; i < n; ++i) state[i] &= 1;
    for (uint32_t k = 0; k < quota && count < R; ++k) {
      uint32_t best = INV;
      for (uint32_t i = 0; i < n; ++i)
        if (!(state[i] & 2) && pickable(i) && has_exact(c, ids[i], label) && better(i, best)) best = i;
      if (best == INV) break;
      state[best] |= 2;
      if (!(state[best] & 1)) {
        state[best] |= 1;
        out_ids[count] = ids[best];
        out_ds[count] = ds[best];
        ++count;
      }
    }
  }
  while (count < R) {
    uint32_t best = INV;
    for (uint32_t i = 0; i < n; ++i)
      if (!(state[i] & 1) && pickable(i) && better(i, best)) best = i;
    if (best == INV) break;
    state[best] |= 1;
    out_ids[count] = ids[best];
    out_ds[count] = ds[best];
    ++count;
  }
  return count;
}

// The publish step for a published degree PR below the build degree R
// (gpu_vamana_filtered.cu:6328-6432): every row's R-row is distanced,
// shortlisted and pruned to PR (canonical_fixed_rare_shortlist :5408-5431 +
// canonical_exact_prune); then rows with reverse edges in that graph are
// rebuilt from their forward row plus new reverse sources, shortlisted and
// pruned to PR again (canonical_reverse_* + canonical_csr_rare_shortlist
// :5433-5450 + canonical_exact_prune).
void publish(const Ctx& c, const std::vector<uint32_t>& ga, const std::vector<uint32_t>& da, uint32_t R,
             uint32_t PR, float alpha, std::vector<uint32_t>& pg, std::vector<uint32_t>& pd) {
  const uint32_t N = c.N;
  pg.assign((size_t)N * PR, INV);
  pd.assign(N, 0);
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t r = 0; r < (int64_t)N; ++r) {
    const uint32_t row = (uint32_t)r, deg = std::min(da[row], R);
    std::vector<uint32_t> ids(ga.begin() + (size_t)row * R, ga.begin() + (size_t)row * R + deg), sid(PR);
    std::vector<float> ds(deg), sd(PR);
    for (uint32_t i = 0; i < deg; ++i) ds[i] = ids[i] < N ? c.D(row, ids[i]) : INFINITY;  // never picked
    const uint32_t n = rare_shortlist(c, row, PR, ids.data(), ds.data(), deg, sid.data(), sd.data());
    pd[row] = filtered_prune(c, row, sid.data(), sd.data(), n, alpha, &pg[(size_t)row * PR], PR);
  }
  std::vector<std::vector<uint32_t>> rev(N);
  for (uint32_t row = 0; row < N; ++row)
    for (uint32_t i = 0; i < std::min(pd[row], PR); ++i) {
      const uint32_t dst = pg[(size_t)row * PR + i];
      if (dst < N && dst != row) rev[dst].push_back(row);
    }
  std::vector<uint32_t> gnew(pg), dnew(pd);
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t r = 0; r < (int64_t)N; ++r) {
    const uint32_t row = (uint32_t)r;
    if (rev[row].empty()) continue;
    const uint32_t deg = std::min(pd[row], PR);
    std::vector<uint32_t> ids(pg.begin() + (size_t)row * PR, pg.begin() + (size_t)row * PR + deg), sid(PR);
    for (uint32_t s : rev[row]) {
      bool dup = s >= N || s == row;
      for (uint32_t i = 0; !dup && i < deg; ++i) dup = pg[(size_t)row * PR + i] == s;
      if (!dup) ids.push_back(s);
    }
    std::vector<float> ds(ids.size()), sd(PR);
    for (size_t i = 0; i < ids.size(); ++i) ds[i] = ids[i] < N ? c.D(row, ids[i]) : INFINITY;
    const uint32_t n = rare_shortlist(c, row, PR, ids.data(), ds.data(), (uint32_t)ids.size(), sid.data(), sd.data());
    dnew[row] = filtered_prune(c, row, sid.data(), sd.data(), n, alpha, &gnew[(size_t)row * PR], PR);
  }
  pg.swap(gnew);
  pd.swap(dnew);
}

// Context with the label -> points postings (ascending rows), as the
// reference builds them on the host (:5753-5765).
Ctx make_ctx(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, const uint32_t* offsets,
             const uint32_t* labels, uint32_t total_labels, const uint32_t* label_starts, uint32_t num_labels,
             uint32_t universal_label) {
  Ctx c{data, dtype, N, dim, R, offsets, labels, num_labels, universal_label, label_starts, {}, {}};
  c.lpo.assign((size_t)std::max(1u, num_labels) + 1, 0);
  for (uint32_t p = 0; p < total_labels; ++p)
    if (labels[p] < num_labels) c.lpo[labels[p] + 1]++;
  for (uint32_t l = 0; l < num_labels; ++l) c.lpo[l + 1] += c.lpo[l];
  c.lpts.assign(c.lpo[num_labels], INV);
  std::vector<uint32_t> cur(c.lpo.begin(), c.lpo.end());
  for (uint32_t row = 0; row < N; ++row)
    for (uint32_t p = offsets[row]; p < offsets[row + 1]; ++p)
      if (labels[p] < num_labels) c.lpts[cur[labels[p]]++] = row;
  return c;
}

}  // namespace

extern "C" {

// filtered_deterministic_random_graph_kernel (:716-744)
void oracle_filtered_random_graph(uint32_t N, uint32_t R, uint32_t initial_degree, uint32_t seed, uint32_t* graph,
                                  uint32_t* degrees) {
  for (uint32_t row = 0; row < N; ++row) {
    const uint32_t target = std::min(std::min(R, initial_degree), N > 0 ? N - 1 : 0u);
    const size_t b = (size_t)row * R;
    uint32_t deg = 0, attempt = 0;
    // the attempt bound (2^20) only guarantees termination
    while (deg < target && attempt < (1u << 20)) {
      const uint32_t cand = fhash(row * 0x9e3779b1u ^ seed * 0x85ebca6bu ^ attempt * 0xc2b2ae35u) % N;
      ++attempt;
      if (cand == row) continue;
      bool dup = false;
      for (uint32_t i = 0; i < deg; ++i) dup |= graph[b + i] == cand;
      if (!dup) graph[b + deg++] = cand;
    }
    for (uint32_t i = deg; i < R; ++i) graph[b + i] = INV;
    degrees[row] = deg;
  }
}

// Per round of the last oracle_filtered_build: changed, touched, reverse proposals.
uint64_t g_round_log[9] = {};

// The last build's per-round counts (9 entries, zero beyond its rounds).
void oracle_filtered_round_log(uint64_t* out) { std::memcpy(out, g_round_log, sizeof(g_round_log)); }

// Full canonical_v2 build. dtype: float input is searched as fp16, so pass
// dtype 2 with rows already rounded to fp16; 1 = uint8. work_C = min(C, 128).
// rounds: canonical rounds (3 in the reference; 0 = random backbone only).
// Returns 0, -1 on bad parameters, 1 when the work buffer cannot hold the
// exact reverse CSR (N*C < 2*N*R).
// diag (optional, 12 entries): invalid, self, low_common, deg_min, deg_max,
// common_min, common_max, out_edges, common_edges, label_checks,
// label_rejects, universal_passes.
int oracle_filtered_build(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t L,
                          uint32_t filtered_L, uint32_t C, uint32_t STEPS, float alpha, const uint32_t* offsets,
                          const uint32_t* labels, uint32_t total_labels, const uint32_t* label_starts,
                          uint32_t num_labels, uint32_t universal_label, uint32_t global_start, uint32_t rounds,
                          uint32_t publish_R, uint32_t* graph_out, uint32_t* degree_out, uint64_t* diag) {
  if (!data || !graph_out || !degree_out || !offsets || !labels || !label_starts) return -1;
  if (N == 0 || dim == 0 || R == 0 || L == 0 || C < R || rounds > 3) return -1;
  const uint32_t work_C = std::min(C, 128u);
  if ((uint64_t)N * work_C < (uint64_t)2 * N * R) return 1;
  Ctx c = make_ctx(data, dtype, N, dim, R, offsets, labels, total_labels, label_starts, num_labels,
                   universal_label);
  std::fill(std::begin(g_round_log), std::end(g_round_log), 0ull);
  const uint32_t per_label_pool = std::min(filtered_L, 32u), per_label_keep = std::min(per_label_pool, 8u);
  const uint32_t ordinary_keep = std::min(R, L), ordinary_pool = std::min(64u, filtered_L);
  std::vector<uint32_t> ga((size_t)N * R), gb((size_t)N * R), da(N), db(N);
  oracle_filtered_random_graph(N, R, std::min(16u, R), 42u, ga.data(), da.data());
  std::vector<uint32_t> task_rows(total_labels);
  for (uint32_t row = 0; row < N; ++row)
    for (uint32_t p = offsets[row]; p < offsets[row + 1]; ++p) task_rows[p] = row;
  std::vector<uint32_t> tids((size_t)total_labels * per_label_keep), work((size_t)N * work_C), wdeg(N);
  std::vector<float> td((size_t)total_labels * per_label_keep), wd((size_t)N * work_C);
  for (uint32_t round = 0; round < rounds; ++round) {
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t p = 0; p < (int64_t)total_labels; ++p)
      task_search(c, ga.data(), da.data(), task_rows[p], labels[p], per_label_pool, per_label_keep, STEPS,
                  &tids[(size_t)p * per_label_keep], &td[(size_t)p * per_label_keep]);
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t r = 0; r < (int64_t)N; ++r)
      ordinary_search(c, ga.data(), da.data(), (uint32_t)r, ordinary_pool, ordinary_keep, STEPS, global_start,
                      &work[(size_t)r * work_C], &wd[(size_t)r * work_C]);
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t r = 0; r < (int64_t)N; ++r) {
      const uint32_t row = (uint32_t)r;
      uint32_t* w = &work[(size_t)row * work_C];
      float* dd = &wd[(size_t)row * work_C];
      wdeg[row] = merge_row(c, ga.data(), da.data(), row, work_C, per_label_keep, ordinary_keep, tids.data(),
                            td.data(), w, dd);
      for (uint32_t i = 0; i < wdeg[row]; ++i)  // canonical_compute_work_distances (:4844-4871)
        if (dd[i] == FLT_MAX) dd[i] = c.D(row, w[i]);
      db[row] = filtered_prune(c, row, w, dd, wdeg[row], alpha, &gb[(size_t)row * R], R);
    }
    // Exact CSR reverse (:4996-5128) + CSR prune (:5130-5230).
    std::vector<std::vector<uint32_t>> rev(N);
    for (uint32_t row = 0; row < N; ++row)
      for (uint32_t i = 0; i < std::min(db[row], R); ++i) {
        const uint32_t dst = gb[(size_t)row * R + i];
        if (dst < N && dst != row) rev[dst].push_back(row);
      }
    std::vector<uint32_t> gnew(gb), dnew(db);
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t r = 0; r < (int64_t)N; ++r) {
      const uint32_t row = (uint32_t)r;
      if (rev[row].empty()) continue;
      const uint32_t deg = std::min(db[row], R);
      std::vector<uint32_t> ids(gb.begin() + (size_t)row * R, gb.begin() + (size_t)row * R + deg);
      for (uint32_t s : rev[row]) {
        bool dup = s >= N || s == row;
        for (uint32_t i = 0; !dup && i < deg; ++i) dup = gb[(size_t)row * R + i] == s;
        if (!dup) ids.push_back(s);
      }
      std::vector<float> ds(ids.size());
      for (size_t i = 0; i < ids.size(); ++i) ds[i] = c.D(row, ids[i]);
      dnew[row] = filtered_prune(c, row, ids.data(), ds.data(), (uint32_t)ids.size(), alpha, &gnew[(size_t)row * R],
                                 R);
    }
    // The round line's counts (gpu_vamana_filtered.cu:6106-6297): rows whose
    // row set or degree changed against the round's input, rows with a
    // reverse source, reverse proposals.
    uint64_t changed = 0, touched = 0, proposals = 0;
    for (uint32_t row = 0; row < N; ++row) {
      touched += !rev[row].empty();
      proposals += rev[row].size();
      const uint32_t od = std::min(da[row], R), nd = std::min(dnew[row], R);
      bool ch = od != nd;
      for (uint32_t i = 0; !ch && i < nd; ++i) {
        bool found = false;
        for (uint32_t k = 0; !found && k < od; ++k) found = ga[(size_t)row * R + k] == gnew[(size_t)row * R + i];
        ch = !found;
      }
      changed += ch;
    }
    g_round_log[3 * round] = changed;
    g_round_log[3 * round + 1] = touched;
    g_round_log[3 * round + 2] = proposals;
    ga.swap(gnew);
    da.swap(dnew);
  }
  if (publish_R > 0 && publish_R < R) {
    std::vector<uint32_t> pg, pd;
    publish(c, ga, da, R, publish_R, alpha, pg, pd);
    ga.swap(pg);
    da.swap(pd);
    R = publish_R;
  }
  std::memcpy(graph_out, ga.data(), ga.size() * 4);
  std::memcpy(degree_out, da.data(), da.size() * 4);
  if (diag) {
    uint64_t invalid = 0, self = 0, low = 0, dmin = 0xFFFFFFFFu, dmax = 0, cmin = 0xFFFFFFFFu, cmax = 0, oe = 0, ce = 0;
    uint64_t checks = 0, uni = 0;
    for (uint32_t row = 0; row < N; ++row) {
      const uint32_t deg = da[row];
      dmin = std::min<uint64_t>(dmin, deg);
      dmax = std::max<uint64_t>(dmax, deg);
      oe += deg;
      uint32_t common = 0;
      for (uint32_t j = 0; j < deg && j < R; ++j) {
        const uint32_t nb = ga[(size_t)row * R + j];
        if (nb == INV || nb >= N) { ++invalid; continue; }
        if (nb == row) { ++self; continue; }
        ++checks;
        // has_common with the universal rule, noting universal passes
        uint32_t i = offsets[row], k = offsets[nb];
        while (i < offsets[row + 1] && k < offsets[nb + 1]) {
          const uint32_t x = labels[i], y = labels[k];
          if (x == universal_label || y == universal_label) { ++uni; ++common; break; }
          if (x == y) { ++common; break; }
          if (x < y) ++i; else ++k;
        }
      }
      ce += common;
      cmin = std::min<uint64_t>(cmin, common);
      cmax = std::max<uint64_t>(cmax, common);
      if (common < 2) ++low;
    }
    const uint64_t v[12] = {invalid, self, low, dmin, dmax, cmin, cmax, oe, ce, checks, checks - ce, uni};
    std::memcpy(diag, v, sizeof(v));
  }
  return 0;
}

// Pinning hook (tests only): one rare-label shortlist of an explicit list.
uint32_t oracle_filtered_shortlist(uint32_t N, uint32_t R, const uint32_t* offsets, const uint32_t* labels,
                                   uint32_t total_labels, uint32_t num_labels, uint32_t universal, uint32_t row,
                                   const uint32_t* ids, const float* ds, uint32_t n, uint32_t* out_ids,
                                   float* out_ds) {
  std::vector<uint32_t> starts(std::max(1u, num_labels), INV);
  Ctx c = make_ctx(nullptr, 1, N, 1, R, offsets, labels, total_labels, starts.data(), num_labels, universal);
  return rare_shortlist(c, row, R, ids, ds, n, out_ids, out_ds);
}

// Pinning hooks (tests only): one FilteredRobustPrune of an explicit list,
// and one merge + label quota of explicit task / old-neighbour / union inputs.
uint32_t oracle_filtered_prune(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, float alpha,
                               const uint32_t* offsets, const uint32_t* labels, uint32_t row, const uint32_t* ids,
                               const float* ds, uint32_t n, uint32_t* out) {
  Ctx c{data, dtype, N, dim, R, offsets, labels, 0, INV, nullptr, {}, {}};
  return filtered_prune(c, row, ids, ds, n, alpha, out, R);
}

uint32_t oracle_filtered_merge(uint32_t N, uint32_t R, uint32_t C, uint32_t per_label_keep, const uint32_t* offsets,
                               const uint32_t* labels, uint32_t total_labels, uint32_t num_labels,
                               const uint32_t* graph, const uint32_t* degrees, uint32_t row,
                               const uint32_t* task_ids, const float* task_d, const uint32_t* ord_ids,
                               const float* ord_d, uint32_t ordinary_keep, uint32_t* out_ids, float* out_d) {
  std::vector<uint32_t> starts(std::max(1u, num_labels), INV);
  Ctx c = make_ctx(nullptr, 0, N, 1, R, offsets, labels, total_labels, starts.data(), num_labels, INV);
  for (uint32_t i = 0; i < C; ++i) {
    out_ids[i] = i < ordinary_keep ? ord_ids[i] : INV;
    out_d[i] = i < ordinary_keep ? ord_d[i] : FLT_MAX;
  }
  return merge_row(c, graph, degrees, row, C, per_label_keep, ordinary_keep, task_ids, task_d, out_ids, out_d);
}

// Pinning hooks (tests only): one per-label task search and one union
// (ordinary) search over an explicit graph.
void oracle_filtered_task_search(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R,
                                 const uint32_t* offsets, const uint32_t* labels, uint32_t total_labels,
                                 const uint32_t* starts, uint32_t num_labels, uint32_t universal,
                                 const uint32_t* graph, const uint32_t* degrees, uint32_t row, uint32_t label,
                                 uint32_t pool_cap, uint32_t keep, uint32_t steps, uint32_t* out_ids,
                                 float* out_d) {
  Ctx c = make_ctx(data, dtype, N, dim, R, offsets, labels, total_labels, starts, num_labels, universal);
  task_search(c, graph, degrees, row, label, pool_cap, keep, steps, out_ids, out_d);
}

void oracle_filtered_ordinary_search(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R,
                                     const uint32_t* offsets, const uint32_t* labels, uint32_t total_labels,
                                     const uint32_t* starts, uint32_t num_labels, const uint32_t* graph,
                                     const uint32_t* degrees, uint32_t row, uint32_t pool_cap, uint32_t keep,
                                     uint32_t steps, uint32_t global_start, uint32_t* out_ids, float* out_d) {
  Ctx c = make_ctx(data, dtype, N, dim, R, offsets, labels, total_labels, starts, num_labels, INV);
  ordinary_search(c, graph, degrees, row, pool_cap, keep, steps, global_start, out_ids, out_d);
}

}  // extern "C"
