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
//    DiskANN's OpenMP build, so its output depends on thread timing (one
//    thread gives the deterministic id-order build). Its RobustPrune
//    (oracle_cpu_occlude) and greedy search (oracle_cpu_greedy) are also
//    exported alone; tests/test_cpu_vamana.py pins all three against an
//    independent Python statement of the paper's rules.
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
#include <vector>
#include <omp.h>
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#endif

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

// Row access for the baselines (element type 0 fp32, 1 uint8, 2 fp16).
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
  inline void prefetch(size_t row) const {
    const size_t bytes = (size_t)dim * (dtype == 0 ? 4 : dtype == 1 ? 1 : 2);
    const char* r = (const char*)p + row * bytes;
    for (size_t off = 0; off < bytes; off += 64) __builtin_prefetch(r + off, 0, 3);
  }
};

// Squared L2 for the baselines, which need a fast, good distance, not the
// canonical GPU order.
#if defined(__AVX2__) && defined(__FMA__)
// SIMD squared L2, as DiskANN's distance functions (AVX2 fp32 with fused
// multiply-add; uint8 through 16-bit differences and pairwise madd, exact).
inline float l2_f32(const float* x, const float* y, uint32_t dim) {
  __m256 acc = _mm256_setzero_ps();
  uint32_t e = 0;
  for (; e + 8 <= dim; e += 8) {
    const __m256 t = _mm256_sub_ps(_mm256_loadu_ps(x + e), _mm256_loadu_ps(y + e));
    acc = _mm256_fmadd_ps(t, t, acc);
  }
  __m128 h = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
  h = _mm_hadd_ps(h, h);
  h = _mm_hadd_ps(h, h);
  float s = _mm_cvtss_f32(h);
  for (; e < dim; ++e) {
    const float t = x[e] - y[e];
    s += t * t;
  }
  return s;
}
inline float l2_u8(const uint8_t* x, const uint8_t* y, uint32_t dim) {
  __m256i acc = _mm256_setzero_si256();
  uint32_t e = 0;
  for (; e + 16 <= dim; e += 16) {
    const __m256i a = _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i*)(x + e)));
    const __m256i b = _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i*)(y + e)));
    const __m256i t = _mm256_sub_epi16(a, b);
    acc = _mm256_add_epi32(acc, _mm256_madd_epi16(t, t));
  }
  alignas(32) int32_t part[8];
  _mm256_store_si256((__m256i*)part, acc);
  int64_t s = 0;
  for (int i = 0; i < 8; ++i) s += part[i];
  for (; e < dim; ++e) {
    const int t = (int)x[e] - (int)y[e];
    s += t * t;
  }
  return (float)s;
}
#else
inline float l2_f32(const float* x, const float* y, uint32_t dim) {
  float s = 0.f;
  for (uint32_t e = 0; e < dim; ++e) {
    const float t = x[e] - y[e];
    s += t * t;
  }
  return s;
}
inline float l2_u8(const uint8_t* x, const uint8_t* y, uint32_t dim) {
  int64_t s = 0;
  for (uint32_t e = 0; e < dim; ++e) {
    const int t = (int)x[e] - (int)y[e];
    s += t * t;
  }
  return (float)s;
}
#endif

inline float l2(const Vecs& A, size_t a, const Vecs& B, size_t b) {
  const uint32_t dim = A.dim;
  if (A.dtype == 0 && B.dtype == 0)
    return l2_f32((const float*)A.p + a * dim, (const float*)B.p + b * dim, dim);
  if (A.dtype == 1 && B.dtype == 1)
    return l2_u8((const uint8_t*)A.p + a * dim, (const uint8_t*)B.p + b * dim, dim);
  float s = 0.f;
  for (uint32_t e = 0; e < dim; ++e) {
    float t = A.elem(a, e) - B.elem(b, e);
    s += t * t;
  }
  return s;
}

// Per-point lock of the CPU build (DiskANN locks each point's row the same
// way): a test-and-set flag, held only while a row is copied or written.
struct SpinLock {
  std::atomic_flag f = ATOMIC_FLAG_INIT;
  void lock() {
    while (f.test_and_set(std::memory_order_acquire)) {
#if defined(__x86_64__)
      __builtin_ia32_pause();
#endif
    }
  }
  void unlock() { f.clear(std::memory_order_release); }
};

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
    // the unvisited neighbours first, their rows prefetched, then the
    // distances (DiskANN's iterate_to_fixed_point gathers and prefetches the
    // same way: the rows are random DRAM reads once the base outgrows the
    // caches)
    size_t fresh = 0;
    for (uint32_t n : tmp) {
      if (seen[n]) continue;
      seen[n] = 1;
      seen_list.push_back(n);
      tmp[fresh++] = n;
      base.prefetch(n);
    }
    for (size_t k = 0; k < fresh; ++k) {
      const uint32_t n = tmp[k];
      beam.insert({l2(q, qrow, base, n), n});
    }
    if (ndist) *ndist += fresh;
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
// DiskANN's calculate_entry_point). threads <= 0 uses every OpenMP thread;
// with 1 thread the points are inserted in id order and the graph is
// deterministic.
//
// Per point p, in id order over the threads (Alg. 1 of the paper, one pass
// at the given alpha):
//   1. greedy search for p from the start with a beam of L; V = the
//      expanded points;
//   2. RobustPrune(p, V \ {p}) (pool = 0: DiskANN's
//      search_for_point_and_prune, which prunes the expanded set and
//      overwrites the row) or RobustPrune(p, V u N_out(p) \ {p}) (pool = 1:
//      the paper's Alg. 2, which keeps the reverse edges p received so far
//      among the candidates); candidates sorted by (distance, id), repeated
//      ids dropped, the occlude alpha ladder; the result becomes N_out(p);
//   3. for every n in N_out(p) without p: append p while n holds fewer than
//      ceil(1.3 R) neighbours (DiskANN's graph slack), else RobustPrune(n,
//      N_out(n) u {p}).
// A last pass prunes rows still above R. Rows live in flat N x max(slack, R)
// arrays with a spinlock per point, so the search copies a neighbour row
// without allocating.
uint32_t oracle_cpu_vamana_build(const void* data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t L,
                                 float alpha, uint32_t maxc, int threads, int pool, uint32_t* graph_out,
                                 uint32_t* degree_out) {
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
  const uint32_t cap = std::max(slack, R);
  // DANCE_ORACLE_PROGRESS set: a line on stderr per tenth of the points inserted
  const bool progress = std::getenv("DANCE_ORACLE_PROGRESS") != nullptr;
  const uint64_t tick = std::max<uint64_t>(1, N / 10);
  std::atomic<uint64_t> inserted{0};
  std::vector<uint32_t> adj((size_t)N * cap);
  std::vector<uint32_t> deg(N, 0);
  std::vector<SpinLock> locks(N);
  const int nt = threads > 0 ? threads : omp_get_max_threads();
  std::vector<std::vector<uint8_t>> seen(nt, std::vector<uint8_t>(N, 0));
  auto row = [&](uint32_t u) { return adj.data() + (size_t)u * cap; };
  // RobustPrune of n over ids (n itself and repeats dropped) into n's row
  auto prune_into = [&](uint32_t n, const uint32_t* ids, uint32_t count, std::vector<Cand>& cp,
                        std::vector<uint32_t>& np) {
    cp.clear();
    for (uint32_t i = 0; i < count; ++i)
      if (ids[i] != n) cp.push_back({l2(base, n, base, ids[i]), ids[i]});
    std::sort(cp.begin(), cp.end());
    cp.erase(std::unique(cp.begin(), cp.end(), [](const Cand& a, const Cand& b) { return a.id == b.id; }),
             cp.end());
    occlude(base, cp, R, alpha, maxc, np);
  };
#pragma omp parallel for schedule(dynamic, 64) num_threads(nt)
  for (int64_t nn = 0; nn < (int64_t)N; ++nn) {
    const uint32_t node = (uint32_t)nn;
    const int tid = omp_get_thread_num();
    std::vector<uint32_t> seen_list, ids, copy, pruned, np;
    std::vector<Cand> cand, cp;
    Beam beam(L);
    auto nbrs = [&](uint32_t u, std::vector<uint32_t>& out) {
      locks[u].lock();
      out.assign(row(u), row(u) + deg[u]);
      locks[u].unlock();
    };
    greedy(base, base, node, start, L, nbrs, seen[tid], seen_list, &cand, beam, nullptr);
    for (uint32_t s : seen_list) seen[tid][s] = 0;
    ids.clear();
    for (const Cand& c : cand) ids.push_back(c.id);
    if (pool == 1) {
      locks[node].lock();
      ids.insert(ids.end(), row(node), row(node) + deg[node]);
      locks[node].unlock();
    }
    prune_into(node, ids.data(), (uint32_t)ids.size(), cp, pruned);
    locks[node].lock();
    std::copy(pruned.begin(), pruned.end(), row(node));
    deg[node] = (uint32_t)pruned.size();
    locks[node].unlock();
    for (uint32_t n : pruned) {
      locks[n].lock();
      const uint32_t* r = row(n);
      if (std::find(r, r + deg[n], node) != r + deg[n]) {
        locks[n].unlock();
        continue;
      }
      if (deg[n] < slack) {
        row(n)[deg[n]++] = node;
        locks[n].unlock();
        continue;
      }
      copy.assign(r, r + deg[n]);
      locks[n].unlock();
      copy.push_back(node);
      prune_into(n, copy.data(), (uint32_t)copy.size(), cp, np);
      locks[n].lock();
      std::copy(np.begin(), np.end(), row(n));
      deg[n] = (uint32_t)np.size();
      locks[n].unlock();
    }
    const uint64_t done = inserted.fetch_add(1) + 1;
    if (progress && done % tick == 0)
      std::fprintf(stderr, "[cpu_vamana] %llu / %u points inserted\n", (unsigned long long)done, N);
  }
#pragma omp parallel for schedule(dynamic, 256) num_threads(nt)
  for (int64_t nn = 0; nn < (int64_t)N; ++nn) {
    const uint32_t n = (uint32_t)nn;
    if (deg[n] > R) {
      std::vector<Cand> cp;
      std::vector<uint32_t> np;
      prune_into(n, row(n), deg[n], cp, np);
      std::copy(np.begin(), np.end(), row(n));
      deg[n] = (uint32_t)np.size();
    }
    const uint32_t k = std::min(deg[n], R);
    degree_out[n] = k;
    for (uint32_t i = 0; i < R; ++i) graph_out[(size_t)n * R + i] = i < k ? row(n)[i] : INV;
  }
  return start;
}

// RobustPrune alone (the occlude step of the build above): candidates
// (ids[i], dists[i]) of point p, sorted by (distance, id) here, cut to maxc,
// then the alpha ladder. Writes at most R ids to out and returns the count.
uint32_t oracle_cpu_occlude(const void* data, int dtype, uint32_t dim, const uint32_t* ids, const float* dists,
                            uint32_t count, uint32_t R, float alpha, uint32_t maxc, uint32_t* out) {
  Vecs base{data, dtype, dim};
  std::vector<Cand> pool(count);
  for (uint32_t i = 0; i < count; ++i) pool[i] = {dists[i], ids[i]};
  std::sort(pool.begin(), pool.end());
  std::vector<uint32_t> res;
  occlude(base, pool, R, alpha, maxc, res);
  std::copy(res.begin(), res.end(), out);
  return (uint32_t)res.size();
}

// The build's greedy search alone, over an N x R graph (INV-padded rows with
// degrees) for query row qrow of `queries`: writes the expanded ids in
// expansion order (at most N) and returns their count; beam_ids (L entries,
// INV-padded) gets the final beam.
uint32_t oracle_cpu_greedy(const void* data, int dtype, uint32_t N, uint32_t dim, const uint32_t* graph,
                           const uint32_t* degree, uint32_t R, uint32_t start, const void* queries, uint32_t qrow,
                           uint32_t L, uint32_t* expanded_out, uint32_t* beam_ids) {
  Vecs base{data, dtype, dim}, qv{queries, dtype, dim};
  std::vector<uint8_t> seen(N, 0);
  std::vector<uint32_t> seen_list;
  std::vector<Cand> exp;
  Beam beam(L);
  auto nbrs = [&](uint32_t u, std::vector<uint32_t>& out) {
    const uint32_t d = std::min(degree[u], R);
    for (uint32_t i = 0; i < d; ++i) {
      const uint32_t v = graph[(size_t)u * R + i];
      if (v < N) out.push_back(v);
    }
  };
  greedy(base, qv, qrow, start, L, nbrs, seen, seen_list, &exp, beam, nullptr);
  for (size_t i = 0; i < exp.size(); ++i) expanded_out[i] = exp[i].id;
  for (uint32_t i = 0; i < L; ++i) beam_ids[i] = i < beam.v.size() ? beam.v[i].id : INV;
  return (uint32_t)exp.size();
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
