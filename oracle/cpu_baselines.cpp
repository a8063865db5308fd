// CPU baselines and evaluators for the GPU Vamana build.
//
// TEST INFRASTRUCTURE ONLY (see vamana_oracle.cpp). Provides:
//  * oracle_cpu_vamana_build: Microsoft DiskANN's in-memory Vamana build
//    restated from its published algorithm (Subramanya et al., "DiskANN",
//    NeurIPS 2019, Alg. 1-3; the occlude_list alpha ladder of DiskANN's
//    Index::prune_neighbors). Upstream DiskANN (commit 78256bba, the base of
//    /root/reference/integrations/dance-diskann-78256bba.patch) cannot be
//    fetched offline, so this restatement stands in as the CPU reference
//    build for recall and timing. It is parallel with per-vertex locks, like
//    DiskANN's OpenMP build, so its output depends on thread timing.
//  * oracle_beam_search: DiskANN search_memory_index semantics (best-first
//    search with a sorted candidate list of size L from the start point).
//  * oracle_bruteforce_knn: exact top-k in double precision, ties by id.

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <vector>
#include <omp.h>

namespace {

constexpr uint32_t INV = 0xFFFFFFFFu;

inline float h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = -1;
      do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
      man &= 0x3FFu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// Plain squared L2 in fp32 (sequential). The baselines need a good distance,
// not the canonical GPU order.
struct Vecs {
  const void* p;
  int dtype;
  uint32_t dim;
  inline float elem(size_t row, uint32_t e) const {
    switch (dtype) {
      case 0: return ((const float*)p)[row * dim + e];
      case 1: return (float)((const uint8_t*)p)[row * dim + e];
      default: return h2f(((const uint16_t*)p)[row * dim + e]);
    }
  }
};

inline float l2(const Vecs& A, size_t a, const Vecs& B, size_t b) {
  const uint32_t dim = A.dim;
  if (A.dtype == 0 && B.dtype == 0) {
    const float* x = (const float*)A.p + a * dim;
    const float* y = (const float*)B.p + b * dim;
    float s = 0.f;
    for (uint32_t e = 0; e < dim; ++e) {
      float t = x[e] - y[e];
      s += t * t;
    }
    return s;
  }
  if (A.dtype == 1 && B.dtype == 1) {
    const uint8_t* x = (const uint8_t*)A.p + a * dim;
    const uint8_t* y = (const uint8_t*)B.p + b * dim;
    int64_t s = 0;
    for (uint32_t e = 0; e < dim; ++e) {
      int t = (int)x[e] - (int)y[e];
      s += t * t;
    }
    return (float)s;
  }
  float s = 0.f;
  for (uint32_t e = 0; e < dim; ++e) {
    float t = A.elem(a, e) - B.elem(b, e);
    s += t * t;
  }
  return s;
}

struct Cand {
  float d;
  uint32_t id;
  bool operator<(const Cand& o) const { return d < o.d || (d == o.d && id < o.id); }
};

// Sorted bounded candidate list (DiskANN NeighborPriorityQueue semantics).
struct Beam {
  uint32_t cap;
  std::vector<Cand> v;
  std::vector<uint8_t> expanded;
  uint32_t cursor = 0;  // first unexpanded position
  explicit Beam(uint32_t L) : cap(L) {
    v.reserve(L + 1);
    expanded.reserve(L + 1);
  }
  void insert(Cand c) {
    if (v.size() == cap && !(c < v.back())) return;
    auto it = std::lower_bound(v.begin(), v.end(), c);
    size_t pos = (size_t)(it - v.begin());
    if (pos < v.size() && v[pos].id == c.id) return;
    v.insert(it, c);
    expanded.insert(expanded.begin() + (long)pos, 0);
    if (v.size() > cap) {
      v.pop_back();
      expanded.pop_back();
    }
    if (pos < cursor) cursor = (uint32_t)pos;
  }
  int next() {
    while (cursor < v.size() && expanded[cursor]) ++cursor;
    if (cursor >= v.size()) return -1;
    expanded[cursor] = 1;
    return (int)cursor;
  }
};

// Greedy best-first search; returns the expanded nodes (the "visited" list of
// DiskANN's search_for_point_and_prune) and fills the final beam.
template <class Neighbors>
void greedy(const Vecs& base, const Vecs& q, size_t qrow, uint32_t start, uint32_t L, Neighbors&& nbrs,
            std::vector<uint8_t>& seen, std::vector<uint32_t>& seen_list, std::vector<Cand>* expanded_out,
            Beam& beam, uint64_t* ndist) {
  beam.v.clear();
  beam.expanded.clear();
  beam.cursor = 0;
  seen[start] = 1;
  seen_list.push_back(start);
  beam.insert({l2(q, qrow, base, start), start});
  if (ndist) ++*ndist;
  std::vector<uint32_t> tmp;
  while (true) {
    int p = beam.next();
    if (p < 0) break;
    Cand c = beam.v[(size_t)p];
    if (expanded_out) expanded_out->push_back(c);
    tmp.clear();
    nbrs(c.id, tmp);
    for (uint32_t n : tmp) {
      if (seen[n]) continue;
      seen[n] = 1;
      seen_list.push_back(n);
      beam.insert({l2(q, qrow, base, n), n});
      if (ndist) ++*ndist;
    }
  }
}

// DiskANN occlude_list: alpha ladder 1.0, 1.2x, ... up to alpha.
void occlude(const Vecs& base, std::vector<Cand>& pool, uint32_t R, float alpha, uint32_t maxc,
             std::vector<uint32_t>& result) {
  result.clear();
  if (pool.size() > maxc) pool.resize(maxc);
  std::vector<float> occ(pool.size(), 0.0f);
  float cur_alpha = 1.0f;
  while (cur_alpha <= alpha && result.size() < R) {
    for (size_t i = 0; i < pool.size() && result.size() < R; ++i) {
      if (occ[i] > cur_alpha) continue;
      occ[i] = FLT_MAX;
      result.push_back(pool[i].id);
      for (size_t j = i + 1; j < pool.size(); ++j) {
        if (occ[j] > alpha) continue;
        float djk = l2(base, pool[i].id, base, pool[j].id);
        occ[j] = (djk == 0.0f) ? FLT_MAX : std::max(occ[j], pool[j].d / djk);
      }
    }
    cur_alpha *= 1.2f;
  }
}

}  // namespace

extern "C" {

// DiskANN-style CPU Vamana build (see file header). graph_out is N x R,
// INV-padded; returns the start point (closest point to the centroid, like
// DiskANN's calculate_entry_point).
uint32_t oracle_cpu_vamana_build(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t L,
                                 float alpha, uint32_t maxc, uint32_t* graph_out, uint32_t* degree_out) {
  Vecs base{data, dtype, dim};
  std::vector<double> centroid(dim, 0.0);
  for (size_t i = 0; i < N; ++i)
    for (uint32_t e = 0; e < dim; ++e) centroid[e] += base.elem(i, e);
  for (uint32_t e = 0; e < dim; ++e) centroid[e] /= (double)N;
  uint32_t start = 0;
  double best = 1e300;
  for (uint32_t i = 0; i < N; ++i) {
    double s = 0;
    for (uint32_t e = 0; e < dim; ++e) {
      double t = base.elem(i, e) - centroid[e];
      s += t * t;
    }
    if (s < best) {
      best = s;
      start = i;
    }
  }
  const uint32_t slack = (uint32_t)std::ceil(1.3 * R);
  // DANCE_ORACLE_PROGRESS set: a line on stderr per tenth of the points inserted
  const bool progress = std::getenv("DANCE_ORACLE_PROGRESS") != nullptr;
  const uint64_t tick = std::max<uint64_t>(1, N / 10);
  std::atomic<uint64_t> inserted{0};
  std::vector<std::vector<uint32_t>> G(N);
  std::vector<std::mutex> locks(N);
  const int nt = omp_get_max_threads();
  std::vector<std::vector<uint8_t>> seen(nt, std::vector<uint8_t>(N, 0));
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t nn = 0; nn < (int64_t)N; ++nn) {
    const uint32_t node = (uint32_t)nn;
    const int tid = omp_get_thread_num();
    std::vector<uint32_t> seen_list;
    std::vector<Cand> pool;
    Beam beam(L);
    auto nbrs = [&](uint32_t u, std::vector<uint32_t>& out) {
      std::lock_guard<std::mutex> lk(locks[u]);
      out = G[u];
    };
    greedy(base, base, node, start, L, nbrs, seen[tid], seen_list, &pool, beam, nullptr);
    for (uint32_t s : seen_list) seen[tid][s] = 0;
    {
      std::lock_guard<std::mutex> lk(locks[node]);
      for (uint32_t u : G[node]) pool.push_back({l2(base, node, base, u), u});
    }
    pool.erase(std::remove_if(pool.begin(), pool.end(), [&](const Cand& c) { return c.id == node; }),
               pool.end());
    std::sort(pool.begin(), pool.end());
    pool.erase(std::unique(pool.begin(), pool.end(), [](const Cand& a, const Cand& b) { return a.id == b.id; }),
               pool.end());
    std::vector<uint32_t> pruned;
    occlude(base, pool, R, alpha, maxc, pruned);
    {
      std::lock_guard<std::mutex> lk(locks[node]);
      G[node] = pruned;
    }
    for (uint32_t n : pruned) {
      std::vector<uint32_t> copy;
      bool need_prune = false;
      {
        std::lock_guard<std::mutex> lk(locks[n]);
        if (std::find(G[n].begin(), G[n].end(), node) != G[n].end()) continue;
        if (G[n].size() < slack) {
          G[n].push_back(node);
          continue;
        }
        copy = G[n];
        copy.push_back(node);
        need_prune = true;
      }
      if (need_prune) {
        std::vector<Cand> cp;
        for (uint32_t u : copy)
          if (u != n) cp.push_back({l2(base, n, base, u), u});
        std::sort(cp.begin(), cp.end());
        std::vector<uint32_t> np;
        occlude(base, cp, R, alpha, maxc, np);
        std::lock_guard<std::mutex> lk(locks[n]);
        G[n] = np;
      }
    }
    const uint64_t done = inserted.fetch_add(1) + 1;
    if (progress && done % tick == 0)
      std::fprintf(stderr, "[cpu_vamana] %llu / %u points inserted\n", (unsigned long long)done, N);
  }
#pragma omp parallel for schedule(dynamic, 256)
  for (int64_t nn = 0; nn < (int64_t)N; ++nn) {
    const uint32_t n = (uint32_t)nn;
    if (G[n].size() > R) {
      std::vector<Cand> cp;
      for (uint32_t u : G[n]) cp.push_back({l2(base, n, base, u), u});
      std::sort(cp.begin(), cp.end());
      std::vector<uint32_t> np;
      occlude(base, cp, R, alpha, maxc, np);
      G[n] = np;
    }
    uint32_t k = (uint32_t)std::min<size_t>(G[n].size(), R);
    degree_out[n] = k;
    for (uint32_t i = 0; i < R; ++i) graph_out[(size_t)n * R + i] = i < k ? G[n][i] : INV;
  }
  return start;
}

// Best-first beam search over an N x R graph (INV-padded rows with degrees).
// ids_out: nq x k. Returns total distance computations.
uint64_t oracle_beam_search(const void* data, int dtype, uint32_t N, uint32_t dim, const uint32_t* graph,
                            const uint32_t* degree, uint32_t R, uint32_t start, const void* queries, uint32_t nq,
                            uint32_t k, uint32_t L, uint32_t* ids_out) {
  Vecs base{data, dtype, dim}, qv{queries, dtype, dim};
  const int nt = omp_get_max_threads();
  std::vector<std::vector<uint8_t>> seen(nt, std::vector<uint8_t>(N, 0));
  uint64_t total = 0;
  if (L < k) L = k;
#pragma omp parallel for schedule(dynamic, 16) reduction(+ : total)
  for (int64_t qq = 0; qq < (int64_t)nq; ++qq) {
    const int tid = omp_get_thread_num();
    std::vector<uint32_t> seen_list;
    Beam beam(L);
    uint64_t nd = 0;
    auto nbrs = [&](uint32_t u, std::vector<uint32_t>& out) {
      uint32_t d = std::min(degree[u], R);
      for (uint32_t i = 0; i < d; ++i) {
        uint32_t v = graph[(size_t)u * R + i];
        if (v < N) out.push_back(v);
      }
    };
    greedy(base, qv, (size_t)qq, start, L, nbrs, seen[tid], seen_list, nullptr, beam, &nd);
    for (uint32_t s : seen_list) seen[tid][s] = 0;
    for (uint32_t i = 0; i < k; ++i) ids_out[(size_t)qq * k + i] = i < beam.v.size() ? beam.v[i].id : INV;
    total += nd;
  }
  return total;
}

// Exact k-NN by brute force in double precision; ties broken by smaller id.
void oracle_bruteforce_knn(const void* data, int dtype, uint32_t N, uint32_t dim, const void* queries, uint32_t nq,
                           uint32_t k, uint32_t* ids_out, float* dists_out) {
  Vecs base{data, dtype, dim}, qv{queries, dtype, dim};
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t qq = 0; qq < (int64_t)nq; ++qq) {
    std::vector<std::pair<double, uint32_t>> best;
    best.reserve(k + 1);
    std::vector<double> q(dim);
    for (uint32_t e = 0; e < dim; ++e) q[e] = qv.elem((size_t)qq, e);
    for (uint32_t i = 0; i < N; ++i) {
      double s = 0;
      for (uint32_t e = 0; e < dim; ++e) {
        double t = q[e] - (double)base.elem(i, e);
        s += t * t;
      }
      std::pair<double, uint32_t> c{s, i};
      if (best.size() < k) {
        best.insert(std::upper_bound(best.begin(), best.end(), c), c);
      } else if (c < best.back()) {
        best.insert(std::upper_bound(best.begin(), best.end(), c), c);
        best.pop_back();
      }
    }
    for (uint32_t i = 0; i < k; ++i) {
      ids_out[(size_t)qq * k + i] = i < best.size() ? best[i].second : INV;
      if (dists_out) dists_out[(size_t)qq * k + i] = i < best.size() ? (float)best[i].first : FLT_MAX;
    }
  }
}

}  // extern "C"
