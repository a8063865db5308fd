// Shard-graph merge on gfx950: diskann::merge_shards_gpu (reference:
// include/gpu_merge.h:8-12, src/gpu_merge.cu:351-790).
//
// The reference expands every shard edge on the host into per-bucket files,
// then sorts and uniques each bucket on the GPU and ranks the edges of a
// source by a 64-bit mix hash. Here the host only reads and parses the shard
// files; everything per edge runs on the device:
//
//   1. k_expand<count>  one wave per shard row: map the row's local neighbours
//      through the shard's id map, drop self loops, flag out-of-range ids, and
//      count the surviving edges of the row's global source (one atomic per row).
//   2. exclusive scan of the counts -> per-source segment offsets.
//   3. k_expand<fill>   same walk; the row reserves its run of the source's
//      segment with one atomic and the lanes write their targets.
//   4. k_rank           one wave per source: the segment's keys
//      (rank << 32 | target) are bitonic-sorted in LDS, duplicates dropped,
//      and the first max_degree targets written back in place. Segments longer
//      than the LDS buffer go through three stable radix sorts instead
//      (target, rank, segment) and k_long_select, with the same result.
//   5. scan of (1 + degree) and k_pack build the DiskANN row bytes
//      (degree, neighbours) of the bucket, which the host writes out.
//
// The order of a source's output row is (rank, target) ascending over its
// distinct targets, which is the reference's order: thrust::sort + unique
// leaves (src, dst) ascending, and its stable sort by (src << 32 | rank)
// breaks rank ties by target (gpu_merge.cu:583-607, 674-681).
//
// Shard bodies stay resident in HBM when they fit beside the bucket buffers
// (one read of every file); otherwise each pass re-uploads them. Buckets split
// the source range only when one bucket would not fit in device memory
// (or DISKANN_GPU_MERGE_BUCKETS / DISKANN_GPU_MERGE_BUCKET_EDGES ask for it);
// the output does not depend on the bucket count.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/dance_hip.h"
#include "../../include/gpu_merge.h"
#include "host_common.h"

namespace dance {
namespace merge {

constexpr uint32_t kWaves = 4;
constexpr uint32_t kBlock = 64 * kWaves;
constexpr uint32_t kBuf = 1024;  // LDS keys per wave (8 KB): segments up to this length sort in LDS
constexpr uint64_t kDefaultSeed = 0x9e3779b97f4a7c15ull;
constexpr uint64_t kReserveBytes = 4ull << 30;
constexpr uint64_t kMaxBuckets = 65536;
constexpr uint64_t kMaxBucketWords = 1ull << 31;  // u32 offsets and scans inside a bucket

// Rank of edge (src, dst) among its source's edges: the 64-bit finaliser mix
// (xor-shift 33, multiply, twice, xor-shift 33) of (src << 32) ^ dst ^ seed,
// folded to 32 bits. Same function as the reference's hash_edge32
// (gpu_merge.cu:89-98): it decides which edges survive the degree cap.
__host__ __device__ __forceinline__ uint32_t edge_rank(uint32_t src, uint32_t dst, uint64_t seed) {
  uint64_t x = ((uint64_t)src << 32) ^ (uint64_t)dst ^ seed;
  x = (x ^ (x >> 33)) * 0xff51afd7ed558ccdull;
  x = (x ^ (x >> 33)) * 0xc4ceb9fe1a85ec53ull;
  x ^= x >> 33;
  return (uint32_t)(x ^ (x >> 32));
}

struct ExpandArgs {
  const uint32_t* words;    // shard body: per row a degree word then its local neighbours
  const uint32_t* row_off;  // word offset of each row's degree word
  const uint32_t* idmap;    // local -> global id
  uint32_t nrows;           // rows of the shard (= id map entries)
  uint32_t lo, hi;          // bucket source range [lo, hi)
  uint32_t* cnt;            // count pass: edges per bucket source; fill pass: write cursors
  uint32_t* seg;            // fill pass: segment storage
  uint32_t* bad;            // count pass: set when a local neighbour id is out of range
  unsigned long long* loops;  // count pass: self loops of bucket sources, 64 stripes
};

// One wave per shard row. FILL = false counts, FILL = true writes targets.
template <bool FILL>
__global__ __launch_bounds__(kBlock) void k_expand(ExpandArgs a) {
  const uint32_t row = grid_block() * kWaves + wave_index();
  if (row >= a.nrows) return;
  const uint32_t lane = lane_id();
  const uint32_t off = a.row_off[row];
  const uint32_t deg = a.words[off];
  const uint32_t src = a.idmap[row];
  const bool in_bucket = src >= a.lo && src < a.hi;
  bool bad = false;
  uint32_t loops = 0;
  for (uint32_t j0 = 0; j0 < deg; j0 += 64) {
    const uint32_t j = j0 + lane;
    const bool act = j < deg;
    const uint32_t ld = act ? a.words[off + 1u + j] : 0u;
    const bool ok = act && ld < a.nrows;
    bad |= act && !ok;
    const uint32_t dst = ok ? a.idmap[ld] : src;
    const bool self = ok && dst == src;
    const bool keep = ok && !self && in_bucket;
    const uint64_t m = wballot(keep);
    if (!FILL) {
      loops += popc64(wballot(self && in_bucket));
      if (lane == 0 && m) atomicAdd(&a.cnt[src - a.lo], popc64(m));
    } else if (m) {
      uint32_t base = 0;
      if (lane == 0) base = atomicAdd(&a.cnt[src - a.lo], popc64(m));
      base = rdlane_u(base, 0);
      if (keep) a.seg[base + mbcnt64(m)] = dst;
    }
  }
  if (!FILL) {
    if (wballot(bad) && lane == 0) atomicOr(a.bad, 1u);
    if (loops && lane == 0) atomicAdd(&a.loops[row & 63u], (unsigned long long)loops);
  }
}

// Ascending bitonic sort of P (power of two, >= 2) keys in one wave's LDS.
__device__ __forceinline__ void wave_bitonic(uint64_t* b, uint32_t P, uint32_t lane) {
  for (uint32_t k = 2; k <= P; k <<= 1) {
    for (uint32_t j = k >> 1; j > 0; j >>= 1) {
      for (uint32_t t = lane; t < P / 2; t += 64) {
        const uint32_t i = ((t & ~(j - 1u)) << 1) | (t & (j - 1u));
        const uint32_t l = i | j;
        const uint64_t x = b[i], y = b[l];
        const bool asc = (i & k) == 0;
        if ((x > y) == asc) {
          b[i] = y;
          b[l] = x;
        }
      }
      wave_sync();
    }
  }
}

// One wave per bucket source: rank, dedupe and cap its segment in place.
// Writes deg[s] = min(distinct, K) and uniq[s] = distinct; segments longer
// than kBuf are listed for the radix path and left untouched.
__global__ __launch_bounds__(kBlock) void k_rank(const uint32_t* __restrict__ offs, uint32_t* __restrict__ seg,
                                                 uint32_t nodes, uint32_t lo, uint32_t K, uint64_t seed,
                                                 uint32_t* __restrict__ deg, uint32_t* __restrict__ uniq,
                                                 uint32_t* __restrict__ long_list,
                                                 uint32_t* __restrict__ long_count) {
  __shared__ uint64_t lds[kWaves * kBuf];
  const uint32_t w = wave_index();
  const uint32_t s = grid_block() * kWaves + w;
  if (s >= nodes) return;
  const uint32_t lane = lane_id();
  const uint32_t begin = offs[s], len = offs[s + 1] - begin;
  if (len > kBuf) {
    if (lane == 0) long_list[atomicAdd(long_count, 1u)] = s;
    return;
  }
  if (len == 0) {
    if (lane == 0) {
      deg[s] = 0;
      uniq[s] = 0;
    }
    return;
  }
  uint64_t* b = lds + (size_t)w * kBuf;
  uint32_t P = 64;
  while (P < len) P <<= 1;
  const uint32_t src = lo + s;
  for (uint32_t i = lane; i < P; i += 64) {
    uint64_t key = ~0ull;  // pads sort last; no real key equals it (targets < 0xFFFFFFFF)
    if (i < len) {
      const uint32_t d = seg[begin + i];
      key = ((uint64_t)edge_rank(src, d, seed) << 32) | d;
    }
    b[i] = key;
  }
  wave_sync();
  wave_bitonic(b, P, lane);
  uint32_t out = 0;
  for (uint32_t base = 0; base < len; base += 64) {
    const uint32_t i = base + lane;
    const uint64_t v = b[i];
    const uint64_t pv = i ? b[i - 1] : ~0ull;
    const bool keep = i < len && v != pv;
    const uint64_t m = wballot(keep);
    const uint32_t pos = out + mbcnt64(m);
    if (keep && pos < K) seg[begin + pos] = (uint32_t)v;
    out += popc64(m);
  }
  if (lane == 0) {
    deg[s] = out < K ? out : K;
    uniq[s] = out;
  }
}

// Long segments: copy each into the packed arrays (targets, segment ordinal,
// identity index for the sorts).
__global__ __launch_bounds__(kBlock) void k_long_gather(const uint32_t* __restrict__ offs,
                                                        const uint32_t* __restrict__ seg,
                                                        const uint32_t* __restrict__ list,
                                                        const uint32_t* __restrict__ loff, uint32_t nlong,
                                                        uint32_t* __restrict__ ldst, uint32_t* __restrict__ lord,
                                                        uint32_t* __restrict__ keys, uint32_t* __restrict__ idx) {
  const uint32_t k = grid_block() * kWaves + wave_index();
  if (k >= nlong) return;
  const uint32_t s = list[k];
  const uint32_t begin = offs[s], len = offs[s + 1] - begin, o = loff[k];
  for (uint32_t i = lane_id(); i < len; i += 64) {
    const uint32_t d = seg[begin + i];
    ldst[o + i] = d;
    lord[o + i] = k;
    keys[o + i] = d;
    idx[o + i] = o + i;
  }
}

// keys[i] = rank of the edge at packed position idx[i].
__global__ void k_long_rank_keys(const uint32_t* __restrict__ idx, const uint32_t* __restrict__ ldst,
                                 const uint32_t* __restrict__ lord, const uint32_t* __restrict__ list, uint32_t lo,
                                 uint64_t seed, uint32_t n, uint32_t* __restrict__ keys) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t j = idx[i];
  keys[i] = edge_rank(lo + list[lord[j]], ldst[j], seed);
}

// keys[i] = segment ordinal of the edge at packed position idx[i].
__global__ void k_long_ord_keys(const uint32_t* __restrict__ idx, const uint32_t* __restrict__ lord, uint32_t n,
                                uint32_t* __restrict__ keys) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  keys[i] = lord[idx[i]];
}

// One wave per long segment, over its (rank, target)-sorted run of idx:
// dedupe and keep the first K targets, written back into the segment.
__global__ __launch_bounds__(kBlock) void k_long_select(const uint32_t* __restrict__ offs, uint32_t* __restrict__ seg,
                                                        const uint32_t* __restrict__ list,
                                                        const uint32_t* __restrict__ loff, uint32_t nlong,
                                                        const uint32_t* __restrict__ idx,
                                                        const uint32_t* __restrict__ ldst, uint32_t K,
                                                        uint32_t* __restrict__ deg, uint32_t* __restrict__ uniq) {
  const uint32_t k = grid_block() * kWaves + wave_index();
  if (k >= nlong) return;
  const uint32_t lane = lane_id();
  const uint32_t s = list[k];
  const uint32_t begin = offs[s], o = loff[k], len = loff[k + 1] - o;
  uint32_t out = 0;
  for (uint32_t base = 0; base < len; base += 64) {
    const uint32_t i = base + lane;
    const bool act = i < len;
    const uint32_t d = act ? ldst[idx[o + i]] : 0u;
    const bool first = act && (i == 0 || ldst[idx[o + i - 1]] != d);
    const uint64_t m = wballot(first);
    const uint32_t pos = out + mbcnt64(m);
    if (first && pos < K) seg[begin + pos] = d;
    out += popc64(m);
  }
  if (lane == 0) {
    deg[s] = out < K ? out : K;
    uniq[s] = out;
  }
}

// pos[s] = 1 + deg[s] (row words), pos[nodes] = 0; scanned into row offsets.
__global__ void k_row_words(const uint32_t* __restrict__ deg, uint32_t nodes, uint32_t* __restrict__ pos) {
  const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s < nodes) pos[s] = 1u + deg[s];
  if (s == nodes) pos[s] = 0u;
}

// One wave per bucket source: its DiskANN row (degree, neighbours).
__global__ __launch_bounds__(kBlock) void k_pack(const uint32_t* __restrict__ offs, const uint32_t* __restrict__ seg,
                                                 const uint32_t* __restrict__ deg, const uint32_t* __restrict__ pos,
                                                 uint32_t nodes, uint32_t* __restrict__ body) {
  const uint32_t s = grid_block() * kWaves + wave_index();
  if (s >= nodes) return;
  const uint32_t lane = lane_id();
  const uint32_t d = deg[s], p = pos[s], o = offs[s];
  if (lane == 0) body[p] = d;
  for (uint32_t j = lane; j < d; j += 64) body[p + 1u + j] = seg[o + j];
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct Shard {
  std::string graph_path, idmap_path;
  std::vector<uint32_t> idmap;
  uint32_t width = 0, medoid = 0;
  uint64_t frozen = 0;
  uint64_t body_words = 0;             // words after the 24-byte header (file size / 4, rounded down)
  std::vector<uint32_t> words;         // body, kept on the host only when not resident
  std::vector<uint32_t> row_off;       // word offset of each row's degree word
  DevBuf d_idmap, d_words, d_row_off;  // device copies (words/row_off only when resident)
};

static uint64_t file_bytes(const std::string& path) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) return UINT64_MAX;
  std::fseek(f, 0, SEEK_END);
  const long n = std::ftell(f);
  std::fclose(f);
  return n < 0 ? UINT64_MAX : (uint64_t)n;
}

// DiskANN .bin of one u32 column (reference read_u32_bin_1d, gpu_merge.cu:62-76).
static bool read_idmap(const std::string& path, std::vector<uint32_t>& out) {
  const uint64_t size = file_bytes(path);
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) return false;
  uint32_t hdr[2] = {0, 0};
  bool ok = std::fread(hdr, 4, 2, f) == 2 && hdr[1] == 1 && size == 8ull + 4ull * hdr[0];
  if (ok) {
    out.resize(hdr[0]);
    ok = hdr[0] == 0 || std::fread(out.data(), 4, hdr[0], f) == hdr[0];
  }
  std::fclose(f);
  return ok;
}

static bool read_header(const std::string& path, uint32_t& width, uint32_t& medoid, uint64_t& frozen) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) return false;
  unsigned char h[24];
  const bool ok = std::fread(h, 1, 24, f) == 24;
  std::fclose(f);
  if (!ok) return false;
  std::memcpy(&width, h + 8, 4);
  std::memcpy(&medoid, h + 12, 4);
  std::memcpy(&frozen, h + 16, 8);
  return true;
}

// Reads a shard body and locates its rows; false when the file ends inside a row.
static bool read_body(Shard& sh) {
  sh.words.assign(sh.body_words, 0u);
  FILE* f = std::fopen(sh.graph_path.c_str(), "rb");
  if (!f) return false;
  bool ok = std::fseek(f, 24, SEEK_SET) == 0 &&
            (sh.body_words == 0 || std::fread(sh.words.data(), 4, sh.body_words, f) == sh.body_words);
  std::fclose(f);
  if (!ok) return false;
  const uint64_t n = sh.idmap.size();
  sh.row_off.resize(n);
  uint64_t off = 0;
  for (uint64_t r = 0; r < n; ++r) {
    if (off >= sh.body_words) return false;
    const uint64_t d = sh.words[off];
    if (off + 1 + d > sh.body_words) return false;
    sh.row_off[r] = (uint32_t)off;
    off += 1 + d;
  }
  return true;
}

static uint32_t bucket_begin(uint64_t b, uint64_t nnodes, uint64_t count) {
  return (uint32_t)((b * nnodes + count - 1) / count);
}

static uint64_t env_u64(const char* name, uint64_t dflt, int base = 10) {
  const char* e = std::getenv(name);
  if (!e || !e[0]) return dflt;
  return std::strtoull(e, nullptr, base);
}

struct Result {
  uint64_t nnodes = 0, replicated = 0, input_edges = 0, self_loops = 0, unique_edges = 0, output_edges = 0;
  uint32_t min_degree = 0, max_degree = 0;
  uint64_t buckets = 0, long_segments = 0;
  int resident = 0;
  double read_s = 0, device_ms = 0, write_s = 0, total_s = 0;
};

static inline uint32_t blocks_for(uint64_t items, uint32_t per_block) {
  return (uint32_t)((items + per_block - 1) / per_block);
}

static int run_merge(const std::string& vamana_prefix, const std::string& vamana_suffix,
                     const std::string& idmaps_prefix, const std::string& idmaps_suffix, uint64_t nshards,
                     uint32_t K, const std::string& output_vamana, const std::string& medoids_file, Result& res) {
  const double t0 = now_sec();
  std::vector<Shard> shards(nshards);
  uint64_t nnodes = 0;
  for (uint64_t i = 0; i < nshards; ++i) {
    Shard& sh = shards[i];
    sh.graph_path = vamana_prefix + std::to_string(i) + vamana_suffix;
    sh.idmap_path = idmaps_prefix + std::to_string(i) + idmaps_suffix;
    if (!read_idmap(sh.idmap_path, sh.idmap)) {
      std::fprintf(stderr, "[GPU merge] failed to read idmap: %s\n", sh.idmap_path.c_str());
      return -2;
    }
    for (uint32_t g : sh.idmap) {
      if (g == 0xFFFFFFFFu) {
        std::fprintf(stderr, "[GPU merge] global id 0xFFFFFFFF in %s is not supported\n", sh.idmap_path.c_str());
        return -2;
      }
      nnodes = std::max<uint64_t>(nnodes, (uint64_t)g + 1);
    }
    res.replicated += sh.idmap.size();
    if (!read_header(sh.graph_path, sh.width, sh.medoid, sh.frozen) || sh.frozen != 0) {
      std::fprintf(stderr, "[GPU merge] invalid graph header: %s\n", sh.graph_path.c_str());
      return -3;
    }
    if (sh.medoid >= sh.idmap.size()) {
      std::fprintf(stderr, "[GPU merge] shard medoid out of range: %s\n", sh.graph_path.c_str());
      return -4;
    }
    sh.body_words = (file_bytes(sh.graph_path) - 24) / 4;
    if (sh.body_words >= (1ull << 32)) {
      std::fprintf(stderr, "[GPU merge] shard graph %s has 2^32 or more words\n", sh.graph_path.c_str());
      return -1;
    }
  }
  res.nnodes = nnodes;

  // Parse every body; count the input edges per global source.
  std::vector<uint64_t> src_edges(nnodes + 1, 0);
  uint64_t total_words = 0;
  for (Shard& sh : shards) {
    if (!read_body(sh)) {
      std::fprintf(stderr, "[GPU merge] truncated graph body: %s\n", sh.graph_path.c_str());
      return -6;
    }
    for (size_t r = 0; r < sh.idmap.size(); ++r) {
      const uint32_t d = sh.words[sh.row_off[r]];
      src_edges[sh.idmap[r]] += d;
      res.input_edges += d;
    }
    total_words += sh.body_words + sh.idmap.size();
  }
  res.read_s = now_sec() - t0;

  // Buckets: the fewest that fit device memory and the 32-bit offsets.
  std::vector<uint64_t> cum(nnodes + 1, 0);
  for (uint64_t v = 0; v < nnodes; ++v) cum[v + 1] = cum[v] + src_edges[v];
  size_t free_b = 0, total_b = 0;
  DHIP(hipMemGetInfo(&free_b, &total_b));
  const uint64_t usable = free_b > kReserveBytes ? free_b - kReserveBytes : free_b / 2;
  auto bucket_bytes = [&](uint64_t nodes, uint64_t edges) {
    // per node: counts/offsets, cursors, degree, distinct count, row words,
    // long list and its body word; per edge: segment, body, and at most six
    // long-path arrays (targets, ordinals, two key and two value buffers)
    return 4 * (7 * nodes + 8 * edges) + (1ull << 20);
  };
  auto fits = [&](uint64_t count, uint64_t budget) {
    for (uint64_t b = 0; b < count; ++b) {
      const uint64_t lo = bucket_begin(b, nnodes, count), hi = bucket_begin(b + 1, nnodes, count);
      const uint64_t e = cum[hi] - cum[lo];
      if (e + (hi - lo) + 1 >= kMaxBucketWords || bucket_bytes(hi - lo, e) > budget) return false;
    }
    return true;
  };
  const uint64_t max_count = std::max<uint64_t>(1, std::min<uint64_t>(kMaxBuckets, nnodes));
  uint64_t count = 1;
  const uint64_t forced = env_u64("DISKANN_GPU_MERGE_BUCKETS", 0);
  const uint64_t target_edges = env_u64("DISKANN_GPU_MERGE_BUCKET_EDGES", 0);
  if (forced) {
    count = forced;
  } else if (target_edges) {
    count = std::max<uint64_t>(1, (res.input_edges + target_edges - 1) / target_edges);
  }
  count = std::min(std::max<uint64_t>(count, 1), max_count);
  const uint64_t resident_bytes = 4 * total_words;
  bool resident = fits(count, usable > resident_bytes ? usable - resident_bytes : 0);
  if (!resident) {
    while (count < max_count && !fits(count, usable)) count = std::min(max_count, count * 2);
    if (!fits(count, usable)) {
      std::fprintf(stderr, "[GPU merge] the merge does not fit device memory even with %llu buckets\n",
                   (unsigned long long)count);
      return -1;
    }
  }
  res.buckets = count;
  res.resident = resident ? 1 : 0;
  std::printf("[GPU merge] nshards=%llu nnodes=%llu replicated_nodes=%llu input_edges=%llu bucket_count=%llu "
              "resident_shards=%d\n",
              (unsigned long long)nshards, (unsigned long long)nnodes, (unsigned long long)res.replicated,
              (unsigned long long)res.input_edges, (unsigned long long)count, (int)resident);

  hipStream_t st = nullptr;
  DHIP(hipStreamCreate(&st));
  struct StreamGuard {
    hipStream_t s;
    ~StreamGuard() {
      if (s) (void)hipStreamDestroy(s);
    }
  } guard{st};

  // Id maps always on the device; bodies too when resident.
  uint64_t max_words = 0, max_rows = 0;
  for (Shard& sh : shards) {
    const size_t n = sh.idmap.size();
    max_words = std::max<uint64_t>(max_words, sh.body_words);
    max_rows = std::max<uint64_t>(max_rows, n);
    DCHECK(sh.d_idmap.alloc(4 * std::max<size_t>(n, 1)));
    if (n) DHIP(hipMemcpyAsync(sh.d_idmap.p, sh.idmap.data(), 4 * n, hipMemcpyHostToDevice, st));
    if (resident) {
      DCHECK(sh.d_words.alloc(4 * std::max<uint64_t>(sh.body_words, 1)));
      DCHECK(sh.d_row_off.alloc(4 * std::max<size_t>(n, 1)));
      if (sh.body_words)
        DHIP(hipMemcpyAsync(sh.d_words.p, sh.words.data(), 4 * sh.body_words, hipMemcpyHostToDevice, st));
      if (n) DHIP(hipMemcpyAsync(sh.d_row_off.p, sh.row_off.data(), 4 * n, hipMemcpyHostToDevice, st));
      DHIP(hipStreamSynchronize(st));
      std::vector<uint32_t>().swap(sh.words);
      std::vector<uint32_t>().swap(sh.row_off);
    }
  }
  DevBuf stage_words, stage_rows;
  if (!resident) {
    DCHECK(stage_words.alloc(4 * std::max<uint64_t>(max_words, 1)));
    DCHECK(stage_rows.alloc(4 * std::max<uint64_t>(max_rows, 1)));
  }

  uint64_t max_nodes = 0, max_edges = 0;
  for (uint64_t b = 0; b < count; ++b) {
    const uint64_t lo = bucket_begin(b, nnodes, count), hi = bucket_begin(b + 1, nnodes, count);
    max_nodes = std::max(max_nodes, hi - lo);
    max_edges = std::max(max_edges, cum[hi] - cum[lo]);
  }
  DevBuf d_cnt, d_cur, d_seg, d_deg, d_uniq, d_pos, d_body, d_flags, d_loops, d_long;
  DCHECK(d_cnt.alloc(4 * (max_nodes + 1)));
  DCHECK(d_cur.alloc(4 * (max_nodes + 1)));
  DCHECK(d_seg.alloc(4 * std::max<uint64_t>(max_edges, 1)));
  DCHECK(d_deg.alloc(4 * (max_nodes + 1)));
  DCHECK(d_uniq.alloc(4 * (max_nodes + 1)));
  DCHECK(d_pos.alloc(4 * (max_nodes + 1)));
  DCHECK(d_body.alloc(4 * (max_nodes + max_edges + 1)));
  DCHECK(d_flags.alloc(8));
  DCHECK(d_loops.alloc(64 * 8));
  DCHECK(d_long.alloc(4 * (max_nodes + 1)));
  DHIP(hipMemsetAsync(d_loops.p, 0, 64 * 8, st));
  ScanWorkspace scan_ws;
  SortWorkspace sort_ws;

  hipEvent_t e0 = nullptr, e1 = nullptr;
  DHIP(hipEventCreate(&e0));
  DHIP(hipEventCreate(&e1));
  struct EventGuard {
    hipEvent_t a, b;
    ~EventGuard() {
      (void)hipEventDestroy(a);
      (void)hipEventDestroy(b);
    }
  } eguard{e0, e1};

  auto expand_pass = [&](bool fill, uint32_t lo, uint32_t hi) -> int {
    for (Shard& sh : shards) {
      const uint32_t n = (uint32_t)sh.idmap.size();
      if (n == 0) continue;
      const uint32_t* words = sh.d_words.as<uint32_t>();
      const uint32_t* rows = sh.d_row_off.as<uint32_t>();
      if (!resident) {
        if (sh.body_words)
          DHIP(hipMemcpyAsync(stage_words.p, sh.words.data(), 4 * sh.body_words, hipMemcpyHostToDevice, st));
        DHIP(hipMemcpyAsync(stage_rows.p, sh.row_off.data(), 4ull * n, hipMemcpyHostToDevice, st));
        words = stage_words.as<uint32_t>();
        rows = stage_rows.as<uint32_t>();
      }
      ExpandArgs a{words, rows, sh.d_idmap.as<uint32_t>(), n, lo, hi,
                   fill ? d_cur.as<uint32_t>() : d_cnt.as<uint32_t>(), d_seg.as<uint32_t>(),
                   d_flags.as<uint32_t>(), d_loops.as<unsigned long long>()};
      if (fill)
        hipLaunchKernelGGL(k_expand<true>, grid_dims(blocks_for(n, kWaves), kBlock), dim3(kBlock), 0, st, a);
      else
        hipLaunchKernelGGL(k_expand<false>, grid_dims(blocks_for(n, kWaves), kBlock), dim3(kBlock), 0, st, a);
      DHIP(hipGetLastError());
      if (!resident) DHIP(hipStreamSynchronize(st));  // the staging buffers are reused by the next shard
    }
    return 0;
  };

  FILE* out = nullptr;
  struct FileGuard {
    FILE** f;
    ~FileGuard() {
      if (*f) std::fclose(*f);
    }
  } fguard{&out};
  uint64_t out_size = 24;
  uint32_t min_deg = nnodes ? UINT32_MAX : 0, max_deg = 0;
  const uint64_t seed = env_u64("DISKANN_GPU_MERGE_HASH_SEED", kDefaultSeed);
  std::vector<uint32_t> h_body, h_deg, h_uniq;

  for (uint64_t b = 0; b < count; ++b) {
    const uint32_t lo = bucket_begin(b, nnodes, count), hi = bucket_begin(b + 1, nnodes, count);
    const uint32_t nodes = hi - lo;
    DHIP(hipEventRecord(e0, st));
    DHIP(hipMemsetAsync(d_cnt.p, 0, 4ull * (nodes + 1), st));
    DHIP(hipMemsetAsync(d_flags.p, 0, 8, st));
    DCHECK(expand_pass(false, lo, hi));
    if (b == 0) {
      // Every edge's local id is checked in the first count pass, before any output.
      uint32_t bad = 0;
      DHIP(hipMemcpyAsync(&bad, d_flags.p, 4, hipMemcpyDeviceToHost, st));
      DHIP(hipStreamSynchronize(st));
      if (bad) {
        std::fprintf(stderr, "[GPU merge] local neighbor out of range in a shard\n");
        return -7;
      }
      FILE* mf = std::fopen(medoids_file.c_str(), "wb");
      if (!mf) return -10;
      const uint32_t mh[2] = {(uint32_t)nshards, 1u};
      bool ok = std::fwrite(mh, 4, 2, mf) == 2;
      for (const Shard& sh : shards) {
        const uint32_t g = sh.idmap[sh.medoid];
        ok = ok && std::fwrite(&g, 4, 1, mf) == 1;
      }
      ok = (std::fclose(mf) == 0) && ok;
      if (!ok) return -10;
      out = std::fopen(output_vamana.c_str(), "wb");
      if (!out) return -11;
      const uint32_t medoid = nshards ? shards[nshards - 1].idmap[shards[nshards - 1].medoid] : 0u;
      unsigned char h[24];
      const uint64_t zero = 0;
      std::memcpy(h, &out_size, 8);
      std::memcpy(h + 8, &K, 4);
      std::memcpy(h + 12, &medoid, 4);
      std::memcpy(h + 16, &zero, 8);
      if (std::fwrite(h, 1, 24, out) != 24) return -11;
    }
    if (nodes == 0) continue;
    DCHECK(scan_exclusive(d_cnt.as<uint32_t>(), (size_t)nodes + 1, scan_ws, st));
    DHIP(hipMemcpyAsync(d_cur.p, d_cnt.p, 4ull * nodes, hipMemcpyDeviceToDevice, st));
    DCHECK(expand_pass(true, lo, hi));
    DHIP(hipMemsetAsync(d_flags.p, 0, 8, st));
    uint32_t* long_count = d_flags.as<uint32_t>() + 1;
    hipLaunchKernelGGL(k_rank, grid_dims(blocks_for(nodes, kWaves), kBlock), dim3(kBlock), 0, st, d_cnt.as<uint32_t>(),
                       d_seg.as<uint32_t>(), nodes, lo, K, seed, d_deg.as<uint32_t>(), d_uniq.as<uint32_t>(),
                       d_long.as<uint32_t>(), long_count);
    DHIP(hipGetLastError());
    uint32_t nlong = 0;
    DHIP(hipMemcpyAsync(&nlong, long_count, 4, hipMemcpyDeviceToHost, st));
    DHIP(hipStreamSynchronize(st));
    if (nlong) {
      // Exact path for segments longer than the LDS buffer: stable radix sorts
      // by target, then rank, then segment ordinal.
      res.long_segments += nlong;
      std::vector<uint32_t> list(nlong), offs(nodes + 1);
      DHIP(hipMemcpy(list.data(), d_long.p, 4ull * nlong, hipMemcpyDeviceToHost));
      DHIP(hipMemcpy(offs.data(), d_cnt.p, 4ull * (nodes + 1), hipMemcpyDeviceToHost));
      std::vector<uint32_t> loff(nlong + 1, 0);
      for (uint32_t k = 0; k < nlong; ++k) loff[k + 1] = loff[k] + (offs[list[k] + 1] - offs[list[k]]);
      const uint32_t T = loff[nlong];
      DevBuf d_list, d_loff, d_ldst, d_lord, kb0, kb1, vb0, vb1;
      DCHECK(d_list.alloc(4ull * nlong));
      DCHECK(d_loff.alloc(4ull * (nlong + 1)));
      DCHECK(d_ldst.alloc(4ull * T));
      DCHECK(d_lord.alloc(4ull * T));
      DCHECK(kb0.alloc(4ull * T));
      DCHECK(kb1.alloc(4ull * T));
      DCHECK(vb0.alloc(4ull * T));
      DCHECK(vb1.alloc(4ull * T));
      DHIP(hipMemcpyAsync(d_list.p, list.data(), 4ull * nlong, hipMemcpyHostToDevice, st));
      DHIP(hipMemcpyAsync(d_loff.p, loff.data(), 4ull * (nlong + 1), hipMemcpyHostToDevice, st));
      uint32_t* keys[2] = {kb0.as<uint32_t>(), kb1.as<uint32_t>()};
      uint32_t* vals[2] = {vb0.as<uint32_t>(), vb1.as<uint32_t>()};
      hipLaunchKernelGGL(k_long_gather, grid_dims(blocks_for(nlong, kWaves), kBlock), dim3(kBlock), 0, st,
                         d_cnt.as<uint32_t>(), d_seg.as<uint32_t>(), d_list.as<uint32_t>(),
                         d_loff.as<uint32_t>(), nlong, d_ldst.as<uint32_t>(), d_lord.as<uint32_t>(), keys[0],
                         vals[0]);
      DHIP(hipGetLastError());
      int r = 0;
      DCHECK(radix_sort_pairs(keys, vals, T, bit_length((uint32_t)(nnodes - 1)), sort_ws, st, &r));
      if (r) {
        std::swap(keys[0], keys[1]);
        std::swap(vals[0], vals[1]);
      }
      hipLaunchKernelGGL(k_long_rank_keys, dim3(blocks_for(T, 256)), dim3(256), 0, st, vals[0],
                         d_ldst.as<uint32_t>(), d_lord.as<uint32_t>(), d_list.as<uint32_t>(), lo, seed, T,
                         keys[0]);
      DHIP(hipGetLastError());
      DCHECK(radix_sort_pairs(keys, vals, T, 32, sort_ws, st, &r));
      if (r) {
        std::swap(keys[0], keys[1]);
        std::swap(vals[0], vals[1]);
      }
      hipLaunchKernelGGL(k_long_ord_keys, dim3(blocks_for(T, 256)), dim3(256), 0, st, vals[0],
                         d_lord.as<uint32_t>(), T, keys[0]);
      DHIP(hipGetLastError());
      DCHECK(radix_sort_pairs(keys, vals, T, bit_length(nlong - 1), sort_ws, st, &r));
      if (r) {
        std::swap(keys[0], keys[1]);
        std::swap(vals[0], vals[1]);
      }
      hipLaunchKernelGGL(k_long_select, grid_dims(blocks_for(nlong, kWaves), kBlock), dim3(kBlock), 0, st,
                         d_cnt.as<uint32_t>(), d_seg.as<uint32_t>(), d_list.as<uint32_t>(),
                         d_loff.as<uint32_t>(), nlong, vals[0], d_ldst.as<uint32_t>(), K, d_deg.as<uint32_t>(),
                         d_uniq.as<uint32_t>());
      DHIP(hipGetLastError());
      DHIP(hipStreamSynchronize(st));
    }
    hipLaunchKernelGGL(k_row_words, dim3(blocks_for((uint64_t)nodes + 1, 256)), dim3(256), 0, st,
                       d_deg.as<uint32_t>(), nodes, d_pos.as<uint32_t>());
    DHIP(hipGetLastError());
    DCHECK(scan_exclusive(d_pos.as<uint32_t>(), (size_t)nodes + 1, scan_ws, st));
    hipLaunchKernelGGL(k_pack, grid_dims(blocks_for(nodes, kWaves), kBlock), dim3(kBlock), 0, st, d_cnt.as<uint32_t>(),
                       d_seg.as<uint32_t>(), d_deg.as<uint32_t>(), d_pos.as<uint32_t>(), nodes,
                       d_body.as<uint32_t>());
    DHIP(hipGetLastError());
    DHIP(hipEventRecord(e1, st));
    uint32_t words = 0;
    DHIP(hipMemcpyAsync(&words, d_pos.as<uint32_t>() + nodes, 4, hipMemcpyDeviceToHost, st));
    DHIP(hipStreamSynchronize(st));
    float ms = 0;
    DHIP(hipEventElapsedTime(&ms, e0, e1));
    res.device_ms += ms;
    h_body.resize(words);
    h_deg.resize(nodes);
    h_uniq.resize(nodes);
    DHIP(hipMemcpy(h_body.data(), d_body.p, 4ull * words, hipMemcpyDeviceToHost));
    DHIP(hipMemcpy(h_deg.data(), d_deg.p, 4ull * nodes, hipMemcpyDeviceToHost));
    DHIP(hipMemcpy(h_uniq.data(), d_uniq.p, 4ull * nodes, hipMemcpyDeviceToHost));
    const double tw = now_sec();
    if (std::fwrite(h_body.data(), 4, words, out) != words) return -11;
    res.write_s += now_sec() - tw;
    out_size += 4ull * words;
    for (uint32_t i = 0; i < nodes; ++i) {
      res.output_edges += h_deg[i];
      res.unique_edges += h_uniq[i];
      min_deg = std::min(min_deg, h_deg[i]);
      max_deg = std::max(max_deg, h_deg[i]);
    }
  }
  unsigned long long loops[64];
  DHIP(hipMemcpy(loops, d_loops.p, sizeof(loops), hipMemcpyDeviceToHost));
  for (int i = 0; i < 64; ++i) res.self_loops += loops[i];
  if (std::fseek(out, 0, SEEK_SET) != 0 || std::fwrite(&out_size, 8, 1, out) != 1) return -11;
  const int rc = std::fclose(out);
  out = nullptr;
  if (rc != 0) return -11;
  res.min_degree = nnodes ? min_deg : 0;
  res.max_degree = max_deg;
  res.total_s = now_sec() - t0;
  std::printf("[GPU merge] unique_edges=%llu output_edges=%llu truncated_edges=%llu self_loops=%llu\n",
              (unsigned long long)res.unique_edges, (unsigned long long)res.output_edges,
              (unsigned long long)(res.unique_edges - res.output_edges), (unsigned long long)res.self_loops);
  std::printf("[GPU merge] degree min=%u avg=%g max=%u\n", res.min_degree,
              nnodes ? (double)res.output_edges / (double)nnodes : 0.0, res.max_degree);
  std::printf("[GPU merge] read_seconds=%g device_ms=%g write_seconds=%g merge_seconds=%g\n", res.read_s,
              res.device_ms, res.write_s, res.total_s);
  std::fflush(stdout);
  return 0;
}

static DanceMergeStats g_last_merge{};

}  // namespace merge
}  // namespace dance

using namespace dance;

namespace diskann {

int merge_shards_gpu(const std::string& vamana_prefix, const std::string& vamana_suffix,
                     const std::string& idmaps_prefix, const std::string& idmaps_suffix, uint64_t nshards,
                     uint32_t max_degree, const std::string& output_vamana, const std::string& medoids_file) {
  merge::Result r;
  const int rc = merge::run_merge(vamana_prefix, vamana_suffix, idmaps_prefix, idmaps_suffix, nshards, max_degree,
                                  output_vamana, medoids_file, r);
  DanceMergeStats s{};
  s.nnodes = r.nnodes;
  s.replicated_nodes = r.replicated;
  s.input_edges = r.input_edges;
  s.self_loops = r.self_loops;
  s.unique_edges = r.unique_edges;
  s.output_edges = r.output_edges;
  s.min_degree = r.min_degree;
  s.max_degree = r.max_degree;
  s.buckets = r.buckets;
  s.long_segments = r.long_segments;
  s.resident_shards = (uint32_t)r.resident;
  s.read_seconds = r.read_s;
  s.device_ms = r.device_ms;
  s.write_seconds = r.write_s;
  s.total_seconds = r.total_s;
  merge::g_last_merge = s;
  return rc;
}

}  // namespace diskann

extern "C" {

int dance_merge_shards(const char* vamana_prefix, const char* vamana_suffix, const char* idmaps_prefix,
                       const char* idmaps_suffix, uint64_t nshards, uint32_t max_degree, const char* output_vamana,
                       const char* medoids_file) {
  if (!vamana_prefix || !vamana_suffix || !idmaps_prefix || !idmaps_suffix || !output_vamana || !medoids_file) {
    std::fprintf(stderr, "[GPU merge] null path argument\n");
    return -1;
  }
  return diskann::merge_shards_gpu(vamana_prefix, vamana_suffix, idmaps_prefix, idmaps_suffix, nshards, max_degree,
                                   output_vamana, medoids_file);
}

void dance_merge_get_last_stats(DanceMergeStats* stats) {
  if (stats) *stats = merge::g_last_merge;
}

}  // extern "C"
