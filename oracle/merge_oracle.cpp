// CPU oracle of the shard-graph merge, diskann::merge_shards_gpu
// (reference: src/gpu_merge.cu:351-790, header include/gpu_merge.h:8-12).
//
// TEST INFRASTRUCTURE ONLY: tests/ call it through oracle/oracle.py as the
// checker of the HIP merge; product code never links it.
//
// A sequential restatement of the reference's steps, file for file:
//   validation of id maps and graph headers      (gpu_merge.cu:405-437)
//   pass 1: expand shard rows into global edges,
//           drop self loops, reject bad local ids (gpu_merge.cu:486-528)
//   medoid file, output header                   (gpu_merge.cu:546-577)
//   pass 2: sort + unique the (src, dst) edges, stable sort by
//           (src << 32 | rank), keep the first max_degree per source
//           (gpu_merge.cu:663-717 with truncate_segments_kernel :140-162)
//   final header size                            (gpu_merge.cu:772-776)
// Buckets are not modelled: they only split the source range and do not
// change the output.
//
// Parity status: oracle_mix64 is pinned by its closed-form inverse
// (tests/test_merge_oracle.py); the merge itself by an independent Python
// restatement (sets and sorted()) on random shard sets, and by invariants.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

// The 64-bit finaliser mix (xor-shift 33, multiply, twice, xor-shift 33).
uint64_t mix64(uint64_t x) {
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdULL;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ULL;
  x ^= x >> 33;
  return x;
}

// hash_edge32 (gpu_merge.cu:89-98).
uint32_t edge_hash(uint32_t src, uint32_t dst, uint64_t seed) {
  const uint64_t x = mix64(((uint64_t)src << 32) ^ (uint64_t)dst ^ seed);
  return (uint32_t)(x ^ (x >> 32));
}

bool read_u32_column(const std::string& path, std::vector<uint32_t>& out) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) return false;
  std::fseek(f, 0, SEEK_END);
  const long size = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  uint32_t n = 0, dim = 0;
  bool ok = std::fread(&n, 4, 1, f) == 1 && std::fread(&dim, 4, 1, f) == 1;
  ok = ok && dim == 1 && (uint64_t)size == 8ull + 4ull * n;
  if (ok) {
    out.resize(n);
    ok = n == 0 || std::fread(out.data(), 4, n, f) == n;
  }
  std::fclose(f);
  return ok;
}

}  // namespace

extern "C" {

uint64_t oracle_mix64(uint64_t x) { return mix64(x); }

uint32_t oracle_edge_hash(uint32_t src, uint32_t dst, uint64_t seed) { return edge_hash(src, dst, seed); }

int oracle_merge_shards(const char* vamana_prefix, const char* vamana_suffix, const char* idmaps_prefix,
                        const char* idmaps_suffix, uint64_t nshards, uint32_t max_degree, const char* output_vamana,
                        const char* medoids_file, uint64_t seed, uint64_t* counters /* self_loops, unique, out */) {
  struct Shard {
    std::string graph, idmap_path;
    std::vector<uint32_t> idmap;
    uint32_t width = 0, medoid = 0;
    uint64_t frozen = 0;
  };
  std::vector<Shard> shards(nshards);
  uint64_t nnodes = 0;
  for (uint64_t i = 0; i < nshards; ++i) {
    Shard& s = shards[i];
    s.graph = std::string(vamana_prefix) + std::to_string(i) + vamana_suffix;
    s.idmap_path = std::string(idmaps_prefix) + std::to_string(i) + idmaps_suffix;
    if (!read_u32_column(s.idmap_path, s.idmap)) return -2;
    for (uint32_t g : s.idmap) nnodes = std::max<uint64_t>(nnodes, (uint64_t)g + 1);
    FILE* f = std::fopen(s.graph.c_str(), "rb");
    uint64_t expected = 0;
    bool ok = f && std::fread(&expected, 8, 1, f) == 1 && std::fread(&s.width, 4, 1, f) == 1 &&
              std::fread(&s.medoid, 4, 1, f) == 1 && std::fread(&s.frozen, 8, 1, f) == 1;
    if (f) std::fclose(f);
    if (!ok || s.frozen != 0) return -3;
    if (s.medoid >= s.idmap.size()) return -4;
  }

  // Pass 1.
  std::vector<uint64_t> edges;
  uint64_t self_loops = 0;
  for (uint64_t i = 0; i < nshards; ++i) {
    const Shard& s = shards[i];
    FILE* f = std::fopen(s.graph.c_str(), "rb");
    if (!f) return -3;
    std::fseek(f, 24, SEEK_SET);
    for (uint32_t local = 0; local < s.idmap.size(); ++local) {
      const uint32_t src = s.idmap[local];
      uint32_t degree = 0;
      if (std::fread(&degree, 4, 1, f) != 1) {
        std::fclose(f);
        return -6;
      }
      std::vector<uint32_t> nbrs(degree);
      if (degree && std::fread(nbrs.data(), 4, degree, f) != degree) {
        std::fclose(f);
        return -6;
      }
      for (uint32_t ld : nbrs) {
        if (ld >= s.idmap.size()) {
          std::fclose(f);
          return -7;
        }
        const uint32_t dst = s.idmap[ld];
        if (dst == src) {
          ++self_loops;
          continue;
        }
        edges.push_back(((uint64_t)src << 32) | dst);
      }
    }
    std::fclose(f);
  }

  FILE* mf = std::fopen(medoids_file, "wb");
  if (!mf) return -10;
  const uint32_t mh[2] = {(uint32_t)nshards, 1u};
  std::fwrite(mh, 4, 2, mf);
  uint32_t out_medoid = 0;
  for (uint64_t i = 0; i < nshards; ++i) {
    const uint32_t g = shards[i].idmap[shards[i].medoid];
    std::fwrite(&g, 4, 1, mf);
    if (i == nshards - 1) out_medoid = g;
  }
  std::fclose(mf);

  FILE* out = std::fopen(output_vamana, "wb");
  if (!out) return -11;
  uint64_t size = 24, frozen = 0;
  std::fwrite(&size, 8, 1, out);
  std::fwrite(&max_degree, 4, 1, out);
  std::fwrite(&out_medoid, 4, 1, out);
  std::fwrite(&frozen, 8, 1, out);

  // Pass 2.
  std::sort(edges.begin(), edges.end());
  edges.erase(std::unique(edges.begin(), edges.end()), edges.end());
  struct Ranked {
    uint64_t key;
    uint32_t dst;
  };
  std::vector<Ranked> ranked(edges.size());
  for (size_t i = 0; i < edges.size(); ++i) {
    const uint32_t src = (uint32_t)(edges[i] >> 32), dst = (uint32_t)edges[i];
    ranked[i] = {((uint64_t)src << 32) | edge_hash(src, dst, seed), dst};
  }
  std::stable_sort(ranked.begin(), ranked.end(), [](const Ranked& a, const Ranked& b) { return a.key < b.key; });
  uint64_t output_edges = 0;
  size_t p = 0;
  for (uint64_t v = 0; v < nnodes; ++v) {
    const size_t start = p;
    while (p < ranked.size() && (ranked[p].key >> 32) == v) ++p;
    const uint32_t keep = (uint32_t)std::min<size_t>(p - start, max_degree);
    std::fwrite(&keep, 4, 1, out);
    for (uint32_t j = 0; j < keep; ++j) std::fwrite(&ranked[start + j].dst, 4, 1, out);
    size += 4ull + 4ull * keep;
    output_edges += keep;
  }
  std::fseek(out, 0, SEEK_SET);
  std::fwrite(&size, 8, 1, out);
  std::fclose(out);
  if (counters) {
    counters[0] = self_loops;
    counters[1] = edges.size();
    counters[2] = output_edges;
  }
  return 0;
}

}  // extern "C"
