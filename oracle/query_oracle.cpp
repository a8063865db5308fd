// CPU oracle of the GPU query search (dance_search).
//
// TEST INFRASTRUCTURE ONLY (see vamana_oracle.cpp). Best-first search with a
// candidate list of the L smallest (distance, id) seen so far and an exact
// visited set, DiskANN search_memory_index semantics
// (iterate_to_fixed_point: expand the closest unexpanded candidate until none
// is left; with a label filter, neighbours without the query label are
// skipped before the visited check and the search starts at the label's
// entry point). Distances are the canonical ones of vamana_oracle.cpp, so
// results are comparable bit for bit with the GPU kernel.

#include <algorithm>
#include <cfloat>
#include <cstdint>
#include <vector>
#include <omp.h>

extern "C" float oracle_distance_rows(const void* a, const void* b, int dtype, uint32_t dim);

namespace {

constexpr uint32_t INV = 0xFFFFFFFFu;

struct Cand {
  float d;
  uint32_t id;
  bool operator<(const Cand& o) const { return d < o.d || (d == o.d && id < o.id); }
};

size_t elem_size(int dtype) { return dtype == 0 ? 4 : dtype == 1 ? 1 : 2; }

bool has_label(const uint32_t* off, const uint32_t* lab, uint32_t p, uint32_t l) {
  for (uint32_t i = off[p]; i < off[p + 1]; ++i) {
    if (lab[i] == l) return true;
    if (lab[i] > l) break;
  }
  return false;
}

}  // namespace

extern "C" {

// starts: with start_offsets null, one entry (shared) or nq entries (per
// query); with start_offsets (nq + 1 entries), query q starts from
// starts[start_offsets[q] .. start_offsets[q + 1]) (DiskANN's init_ids of a
// filtered search: the label's start plus its extra starts,
// integrations/dance-diskann-78256bba.patch:20583-20625; they are inserted
// without the label check, ids >= N skipped). labels: optional filter
// (offsets/labels per point, one label per query). Outputs the k best
// (distance, id) in order, INV / FLT_MAX past the end. Returns the number of
// distances computed.
uint64_t oracle_query_search(const void* data, int dtype, uint32_t N, uint32_t dim, const uint32_t* graph,
                             const uint32_t* degree, uint32_t R, const uint32_t* starts, uint32_t nstarts,
                             const uint32_t* start_offsets, const void* queries, uint32_t nq, uint32_t k,
                             uint32_t L, const uint32_t* offsets, const uint32_t* labels, const uint32_t* qlabels,
                             uint32_t* ids_out, float* d_out) {
  const size_t row = (size_t)dim * elem_size(dtype);
  const char* base = (const char*)data;
  const char* qs = (const char*)queries;
  uint64_t total = 0;
#pragma omp parallel for schedule(dynamic, 8) reduction(+ : total)
  for (int64_t q = 0; q < (int64_t)nq; ++q) {
    std::vector<uint8_t> seen(N, 0);
    std::vector<Cand> pool;  // sorted, at most L
    std::vector<uint8_t> ex;
    const void* qv = qs + (size_t)q * row;
    auto dist = [&](uint32_t v) { return oracle_distance_rows(qv, base + (size_t)v * row, dtype, dim); };
    auto insert = [&](Cand c) {
      if (pool.size() == L && !(c < pool.back())) return;
      auto it = std::lower_bound(pool.begin(), pool.end(), c);
      const size_t pos = (size_t)(it - pool.begin());
      pool.insert(it, c);
      ex.insert(ex.begin() + (long)pos, 0);
      if (pool.size() > L) {
        pool.pop_back();
        ex.pop_back();
      }
    };
    const uint32_t ql = qlabels ? qlabels[q] : INV;
    const uint32_t b0 = start_offsets ? start_offsets[q] : (nstarts == 1 ? 0u : (uint32_t)q);
    const uint32_t b1 = start_offsets ? start_offsets[q + 1] : b0 + 1;
    for (uint32_t b = b0; b < b1; ++b) {
      const uint32_t start = starts[b];
      if (start < N && L > 0 && !seen[start]) {
        seen[start] = 1;
        insert({dist(start), start});
        ++total;
      }
    }
    while (true) {
      size_t p = 0;
      while (p < pool.size() && ex[p]) ++p;
      if (p == pool.size()) break;
      ex[p] = 1;
      const uint32_t u = pool[p].id;
      const uint32_t du = std::min(degree[u], R);
      for (uint32_t j = 0; j < du; ++j) {
        const uint32_t v = graph[(size_t)u * R + j];
        if (v >= N) continue;
        if (qlabels && !has_label(offsets, labels, v, ql)) continue;
        if (seen[v]) continue;
        seen[v] = 1;
        insert({dist(v), v});
        ++total;
      }
    }
    for (uint32_t i = 0; i < k; ++i) {
      ids_out[(size_t)q * k + i] = i < pool.size() ? pool[i].id : INV;
      d_out[(size_t)q * k + i] = i < pool.size() ? pool[i].d : FLT_MAX;
    }
  }
  return total;
}

}  // extern "C"
