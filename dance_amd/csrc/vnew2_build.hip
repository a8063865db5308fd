// Host orchestration of the standard GPU Vamana build and the C ABI of
// include/gpu_vamana_builder.h + include/dance_hip.h.
//
// Build = approximate medoid -> hashed R-regular init -> ITERS x
//   (search + online robust insert -> reverse edges (stable radix sort by
//    target) + merge -> RobustPrune, degree fill in the last iteration),
// the schedule of gpu_vamana_build_impl (/root/reference/src/gpu_vamana_vnew2.cu:2170-2855).
//
// Device layout (one allocation each, row-major):
//   rows   N x stride16 x 16 B   vectors, each row zero-padded to 16 B
//   cur    N x R   u32            current graph (INV-padded)
//   work   N x C   u32 + wd N x C f32   candidate rows with distances
//   keys/vals 2 x 2 x N*R u32     reverse-edge radix sort double buffers
//   offs   N+1 u32                reverse CSR offsets
//   qrows  N x 128 B              int8 codes + header for the distance lower
//                                 bound (fp32/fp16 rows of <= 112 dims)
// All kernels run on one stream; stages are timed with HIP events.
//
// Algorithmic bytes reported for the roofline (per kernel, summed over the
// build; V = bytes of one vector row, counted on device by each wave):
//   search: (search_dist + insert_dist) * V + expansions * (4R + 4)
//           + N * (V + 4R + 4 + 16C)            (own vector, cur row, work row r/w)
//           + bound_checks * 128                (quantized rows, when the bound is on)
//   merge : merge_dist * 4 (snapshot distances read) + reverse_edges * 4 + touched_rows * (16C + 8)
//   prune : prune_dist * V + (selected rows) * V + N * 24C + prune_bound_checks * 128
//   reverse (keys + sort): N*R*(4*3) + passes * N*R * 20

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <type_traits>
#include <utility>
#include <vector>

#include "../../include/dance_hip.h"
#include "../../include/gpu_vamana_builder.h"
#include "../../include/gpu_vamana_filtered.h"
#include "host_common.h"
#include "stitched_kernels.h"
#include "vnew2_kernels.h"

static_assert(sizeof(GPUVamanaStats) == 7 * 8 + 6 * 8 + 8 + 8, "GPUVamanaStats layout");
static_assert(offsetof(GPUVamanaStats, distance_computations) == 56, "GPUVamanaStats layout");
static_assert(offsetof(GPUVamanaStats, reverse_csr_seconds) == 104, "GPUVamanaStats layout");
static_assert(offsetof(GPUVamanaStats, selective_active_nodes) == 112, "GPUVamanaStats layout");

namespace dance {

// ---------------------------------------------------------------------------
// Profiles (reference CMake DANCE_PROFILE, patch:2400-2462; effective
// constants of include/gpu_vamana_config.h).
// ---------------------------------------------------------------------------
struct Profile {
  const char* name;
  bool fp16;
  uint32_t heavy_threshold, heavy_sample;
};
constexpr uint32_t kDefaultIters = 4;       // VAMANA_ITERS
// Largest build list L: the search pool holds 16 slots per lane (the
// reference sizes its LDS pool by L, vnew2.cu:193-199, 2221; DiskANN callers
// build with L of several hundred).
constexpr uint32_t kMaxBuildL = 1024;
constexpr uint32_t kMaxIters = DANCE_MAX_ITERS;  // per-iteration arrays of DanceKernelProfile
constexpr float kAlpha = 1.2f;              // VAMANA_ALPHA (last iteration only)
constexpr uint32_t kFinalMinDegree = 64;    // FINAL_MIN_DEGREE
constexpr uint32_t kWarmupSteps = 64;       // WARMUP_EXPAND_STEPS
constexpr uint32_t kCoarseIters = 2;        // COARSE_WARMUP_ITERS
constexpr uint32_t kMedoidCandidates = 1024;
constexpr uint32_t kMedoidSamples = 4096;

static const Profile kProfiles[] = {
    {"QUALITY", false, 0, 0},
    {"FAST_SMALL", true, 0, 0},
    {"PRO6000_100M", true, 256, 384},
    {"FILTERED_PAPER", true, 256, 384},
};

static std::mutex g_mu;
static int g_profile = -1;

static int profile_index_locked() {
  if (g_profile < 0) {
    g_profile = 0;
    if (const char* e = std::getenv("DANCE_PROFILE")) {
      for (int i = 0; i < 4; ++i)
        if (std::strcmp(e, kProfiles[i].name) == 0) g_profile = i;
    }
  }
  return g_profile;
}

static uint32_t g_last_medoid = 0;
static GPUVamanaStats g_last_stats{};
static DanceKernelProfile g_last_prof{};

// The two standard builders of the reference keep their own last-build state
// (gpu_vamana_vnew2.cu and gpu_vamana_uint8.cu each hold a file-static medoid
// and GPUVamanaStats, uint8.cu:2416-2435), so a v8 build leaves the vnew2
// getters untouched and the other way round.
enum class Builder { vnew2, v8 };
static uint32_t g_last_medoid_v8 = 0;
static GPUVamanaStats g_last_stats_v8{};

// The v8 builder (gpu_vamana_uint8.cu) runs the vnew2 kernels' algorithm with
// C-stride double-buffered graphs and has no reverse heavy cap in any profile:
// its reverse_merge_csr_kernel (uint8.cu:1795-1940) takes every reverse
// candidate. Its search (uint8.cu:1123-1540), insert (:817-950), init
// (:1074-1121), medoid (:1040-1072) and prune (:2020-2298) compute what the
// vnew2 ones do; the graph layout changes no result, so the same kernels serve.
static Profile profile_for(Builder b) {
  Profile p = kProfiles[profile_index_locked()];
  if (b == Builder::v8) p.heavy_threshold = p.heavy_sample = 0;
  return p;
}


// ---------------------------------------------------------------------------
// Graph state + per-stage launchers.
// ---------------------------------------------------------------------------
struct State {
  uint32_t N = 0, R = 0, C = 0;
  DevBuf cur, deg_cur, work, deg_work, wd;
  GraphBufs g() {
    return GraphBufs{N, R, C, cur.as<uint32_t>(), deg_cur.as<uint32_t>(), work.as<uint32_t>(),
                     deg_work.as<uint32_t>(), wd.as<float>()};
  }
  int alloc(uint32_t N_, uint32_t R_, uint32_t C_, bool with_cur = true, bool with_deg = true) {
    N = N_;
    R = R_;
    C = C_;
    if (with_cur) DCHECK(cur.alloc((size_t)N * R * 4));
    if (with_deg) DCHECK(deg_cur.alloc((size_t)N * 4));
    DCHECK(work.alloc((size_t)N * C * 4));
    DCHECK(deg_work.alloc((size_t)N * 4));
    DCHECK(wd.alloc((size_t)N * C * 4));
    return 0;
  }
};

static uint32_t round64(uint32_t x) { return (x + 63u) / 64u * 64u; }

static uint32_t wave_grid(uint32_t n) { return (n + kWavesPerBlock - 1) / kWavesPerBlock; }
// Grid for kernels that remap workgroups across XCDs (xcd_block): a multiple
// of 8 workgroups, 2-D beyond 2^32 work-items (grid_dims).
static dim3 xcd_grid(uint32_t n) { return grid_dims(wave_grid(n), kBlock, 8); }

static int launch_medoid(const Rows& rows, hipStream_t s, float* d_scores, uint32_t* d_cands, uint32_t nc,
                         uint32_t ns) {
  const int cpl = pick_cpl(rows.rs.nch);
  return with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
    hipLaunchKernelGGL((k_medoid<decltype(dt)::value, decltype(c)::value>), dim3(wave_grid(nc)), dim3(kBlock), 0, s,
                       rows.rs, rows.N, nc, ns, d_scores, d_cands);
    DHIP(hipGetLastError());
    return 0;
  });
}

static int launch_init(const Rows& rows, GraphBufs g, hipStream_t s) {
  const int cpl = pick_cpl(rows.rs.nch);
  return with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
    hipLaunchKernelGGL((k_init<decltype(dt)::value, decltype(c)::value>), grid_dims(wave_grid(g.N), kBlock), dim3(kBlock), 0, s,
                       rows.rs, g);
    DHIP(hipGetLastError());
    return 0;
  });
}

// Quantized lower bound (qbound.h). DANCE_QBOUND=0 turns it off; otherwise
// the build uses it in the iterations whose bit is set in DANCE_QBOUND_ITERS
// (default kQBoundIters). Results are identical either way.
constexpr uint32_t kQBoundIters = 0x1u;  // first iteration: random graph, HBM-bound
// Without DANCE_QBOUND_ITERS the search also uses it in the last iteration
// when the iteration before it computed more than kQBoundLastMinDist
// candidate distances per expansion: the last iteration (alpha > 1) then
// gathers more rows than the bound's extra work costs. Measured with both
// variants of the last search launch (4 iterations): c1 (isotropic, 49.5
// distances per expansion in iteration 2) 23.6 -> 14.7 ms with the bound; c3
// (26.7) 935 -> 875 ms; c2 (20.1) 54.2 -> 69.3 ms and c2 with fp16 rows
// (20.1) 70.3 -> 85.7 ms, so it stays off there.
constexpr double kQBoundLastMinDist = 24.0;
static bool qbound_iters_adaptive() {
  const char* e = std::getenv("DANCE_QBOUND_ITERS");
  return !(e && e[0]);
}
// The prune uses it in the iterations of DANCE_QBOUND_PRUNE_ITERS (default
// kQBoundPruneIters), and by default also in iteration 1 when iteration 0's
// prune reached more than a quarter of all candidate pairs (its bound checks
// per vertex above C (C - 1) / 8): the bound's one batch then replaces dense
// exact rounds. Measured: iteration 1's prune at c1 (isotropic data, 41% of
// the pairs reached in iteration 0) 7.07 -> 1.05 ms with the bound; at c2 and
// c3 (clustered, 7.6%) 4.46 -> 5.54 and 47.4 -> 57.2 ms, so it stays off there.
constexpr uint32_t kQBoundPruneIters = ~0x2u;  // every iteration but 1 (0, 2 and 3 of the default 4)
static bool qbound_prune_adaptive() {
  const char* e = std::getenv("DANCE_QBOUND_PRUNE_ITERS");
  return !(e && e[0]);
}
static bool qbound_enabled() {
  const char* e = std::getenv("DANCE_QBOUND");
  return !(e && e[0] == '0');
}
static uint32_t env_mask(const char* name, uint32_t def) {
  const char* e = std::getenv(name);
  if (e && e[0]) return (uint32_t)std::strtoul(e, nullptr, 0);
  return def;
}
static uint32_t qbound_iters() { return env_mask("DANCE_QBOUND_ITERS", kQBoundIters); }
// Iterations whose search also bounds the online insert's occlusion pairs
// (where the search bound is on): by default iteration 0 only, whose work
// rows are the random initial graph, so the rows the exact test gathers
// miss the caches. Measured (iteration 0 / build): c3 1249 -> 1211 ms, 3.676
// -> 3.638 s; c2 120.6 -> 108.3 ms, 310 -> 298 ms; c1 13.6 -> 11.5 ms. In the
// last iteration the rows are mostly cache hits and the bound's per-pair
// work costs more than it saves (c3 857 -> 988 ms).
constexpr uint32_t kInsertBoundIters = 0x1u;
static uint32_t insert_bound_iters() { return env_mask("DANCE_INSERT_BOUND_ITERS", kInsertBoundIters); }
static uint32_t qbound_prune_iters() { return env_mask("DANCE_QBOUND_PRUNE_ITERS", kQBoundPruneIters); }

// Builds the code rows for `rows` into buf; returns a disabled set when the
// row type or width has no bound.
static int build_qbound(const Rows& rows, DevBuf& buf, hipStream_t s, QBoundSet* out) {
  *out = QBoundSet{nullptr, 0.0f, 0.0f};
  if (!qbound_enabled() || rows.dtype == DANCE_U8 || rows.dim > kQMaxDim || rows.N == 0) return 0;
  const int cpl = pick_cpl(rows.rs.nch);
  if (cpl < 0) return 0;
  DCHECK(buf.alloc((size_t)rows.N * kQChunks * 16));
  const uint32_t grid = (uint32_t)(((uint64_t)rows.N * 8 + 255) / 256);  // one octet per row
  if (rows.dtype == DANCE_F32)
    hipLaunchKernelGGL(k_quantize<DANCE_F32>, dim3(grid), dim3(256), 0, s, rows.rs, rows.N, rows.dim, buf.as<uint4>());
  else
    hipLaunchKernelGGL(k_quantize<DANCE_F16>, dim3(grid), dim3(256), 0, s, rows.rs, rows.N, rows.dim, buf.as<uint4>());
  DHIP(hipGetLastError());
  const double lane_terms = (double)cpl * (16.0 / elem_bytes(rows.dtype));
  if (rows.dtype == DANCE_F32) {
    *out = QBoundSet{buf.as<uint4>(), (float)(2.0 * (lane_terms + 8.0) * 0x1p-24), 1e-30f};
  } else {  // binary16 differences and squares (see qbound.h)
    *out = QBoundSet{buf.as<uint4>(), (float)(2.0 * (3.0 * 0x1p-11 + (lane_terms + 8.0) * 0x1p-24)),
                     (float)(1e-30 + (double)rows.dim * 0x1p-24)};
  }
  return 0;
}

// insert_bound: with the search bound on, the online insert's occlusion test
// also decides pairs on the code rows (fp32/fp16 rows of at most 3 chunks
// per lane, C <= 128, L <= 128; elsewhere the request is ignored).
// hashed_cur: the first iteration, whose graph is the random initial one: the
// L <= 128 variants recompute expanded vertices' neighbours instead of
// gathering them, and each vertex's own initial row with its distances (the
// build then launches no k_init at L <= 128).
static int launch_search(const Rows& rows, GraphBufs g, uint32_t L, uint32_t steps, float alpha, uint32_t start,
                         const uint32_t* order, VCounters* ctr, const QBoundSet& qb, hipStream_t s,
                         bool insert_bound, bool hashed_cur) {
  const int cpl = pick_cpl(rows.rs.nch);
  const uint32_t Cp = round64(g.C);
  const size_t lds = (size_t)kWavesPerBlock * search_lds_words(Cp) * 4;
  SearchArgs a{rows.rs, g, L, steps, start, alpha, order, ctr, qb};
  if (L > kMaxBuildL) {
    std::fprintf(stderr, "[dance_hip] L=%u exceeds the supported maximum %u\n", L, kMaxBuildL);
    return -1;
  }
  return with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
    constexpr int DT = decltype(dt)::value, CPL = decltype(c)::value;
    // Bounded variants exist only where build_qbound can produce code rows.
    constexpr bool kHasQB = DT != DANCE_U8 && CPL <= 4;
    if constexpr (kHasQB) {
      if (qb.rows && L <= 256) {
        // (fp16 rows of at most 112 dims take 2 chunks per lane)
        if constexpr (CPL <= (DT == DANCE_F16 ? 2 : 3)) {
          if (insert_bound && L <= 128 && g.C <= 128) {  // nA <= C <= 128 fits the open-pair list
            if (hashed_cur)
              hipLaunchKernelGGL((k_search<DT, CPL, 2, true, true, true>), xcd_grid(g.N), dim3(kBlock), lds, s, a, Cp);
            else
              hipLaunchKernelGGL((k_search<DT, CPL, 2, true, true>), xcd_grid(g.N), dim3(kBlock), lds, s, a, Cp);
            DHIP(hipGetLastError());
            return 0;
          }
        }
        if (L <= 128 && hashed_cur)
          hipLaunchKernelGGL((k_search<DT, CPL, 2, true, false, true>), xcd_grid(g.N), dim3(kBlock), lds, s, a, Cp);
        else if (L <= 128)
          hipLaunchKernelGGL((k_search<DT, CPL, 2, true>), xcd_grid(g.N), dim3(kBlock), lds, s, a, Cp);
        else
          hipLaunchKernelGGL((k_search<DT, CPL, 4, true>), xcd_grid(g.N), dim3(kBlock), lds, s, a, Cp);
        DHIP(hipGetLastError());
        return 0;
      }
    }
    // pools above 256 entries (16 slots per lane) run the exact variant only
    if (L <= 128 && hashed_cur)
      hipLaunchKernelGGL((k_search<DT, CPL, 2, false, false, true>), xcd_grid(g.N), dim3(kBlock), lds, s, a, Cp);
    else if (L <= 128)
      hipLaunchKernelGGL((k_search<DT, CPL, 2, false>), xcd_grid(g.N), dim3(kBlock), lds, s, a, Cp);
    else if (L <= 256)
      hipLaunchKernelGGL((k_search<DT, CPL, 4, false>), xcd_grid(g.N), dim3(kBlock), lds, s, a, Cp);
    else
      hipLaunchKernelGGL((k_search<DT, CPL, 16, false>), xcd_grid(g.N), dim3(kBlock), lds, s, a, Cp);
    DHIP(hipGetLastError());
    return 0;
  });
}

// Which prune kernel: in the iterations whose bit is set in
// DANCE_PRUNE_RANK_ITERS (default kPruneRankIters), rows of at most kRankCap
// candidates take k_prune_rank (with the bound's pair decisions from MFMA
// tiles when qb is on); otherwise, and for wider rows, k_prune. Both give the
// same graph. The default follows the per-launch times: for float rows
// (c3) iteration 0 (alpha 1 right after the random graph: few rounds per
// row, so the rank kernel's up-front sort and all-pairs tiles do not pay) is
// fastest with k_prune and the bound, iterations 1-3 with k_prune_rank; uint8
// rows (c4), whose rank kernel takes every pair from Gram tiles, are fastest
// with k_prune_rank in every iteration.
constexpr uint32_t kPruneRankIters = ~0x1u, kPruneRankItersU8 = ~0u;  // from iteration 1 on / all
static uint32_t prune_rank_iters(int dtype) {
  return env_mask("DANCE_PRUNE_RANK_ITERS", dtype == DANCE_U8 ? kPruneRankItersU8 : kPruneRankIters);
}

// uint8 rows in k_prune_rank: every pair's exact distance from MFMA Gram
// tiles (default), or DANCE_PRUNE_GRAM=0 for exact tests inside the rounds.
// Both give the same graph.
static bool prune_gram() {
  const char* e = std::getenv("DANCE_PRUNE_GRAM");
  return !(e && e[0] == '0');
}

static int launch_prune(const Rows& rows, GraphBufs g, uint32_t min_degree, float alpha, const uint32_t* order,
                        VCounters* ctr, const QBoundSet& qb, bool rank_kernel, hipStream_t s) {
  const int cpl = pick_cpl(rows.rs.nch);
  const uint32_t Cp = round64(g.C), Rp = round64(g.R), Cq = (g.C + 31u) / 32u * 32u;
  PruneArgs a{rows.rs, g, min_degree, alpha, order, ctr, qb};
  const bool rank = Cp <= kRankCap && rank_kernel;
  return with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
    constexpr int DT = decltype(dt)::value, CPL = decltype(c)::value;
    constexpr bool kHasQB = DT != DANCE_U8 && CPL <= 4;
    if (rank) {
      if constexpr (kHasQB) {
        if (qb.rows) {
          hipLaunchKernelGGL((k_prune_rank<DT, CPL, kRankBound>), xcd_grid(g.N), dim3(kBlock),
                             (size_t)kWavesPerBlock * prune_rank_lds_words(Cq, true) * 4, s, a, Cq);
          DHIP(hipGetLastError());
          return 0;
        }
      }
      // without code rows the bound is off: uint8 rows take every pair's
      // distance from Gram tiles, other rows test every pair exactly
      a.qb = QBoundSet{nullptr, 0.0f, 0.0f};
      if constexpr (DT == DANCE_U8) {
        if (prune_gram()) {
          hipLaunchKernelGGL((k_prune_rank<DT, CPL, kRankGram>), xcd_grid(g.N), dim3(kBlock),
                             (size_t)kWavesPerBlock * prune_rank_lds_words(Cq, true) * 4, s, a, Cq);
          DHIP(hipGetLastError());
          return 0;
        }
      }
      hipLaunchKernelGGL((k_prune_rank<DT, CPL, kRankExact>), xcd_grid(g.N), dim3(kBlock),
                         (size_t)kWavesPerBlock * prune_rank_lds_words(Cq, false) * 4, s, a, Cq);
      DHIP(hipGetLastError());
      return 0;
    }
    hipLaunchKernelGGL((k_prune<DT, CPL>), xcd_grid(g.N), dim3(kBlock),
                       (size_t)kWavesPerBlock * prune_lds_words(Cp, Rp) * 4, s, a, Cp, Rp);
    DHIP(hipGetLastError());
    return 0;
  });
}

// The reverse sort's items (forward slots) per part: below 2^32, so that
// its items and offsets stay 32-bit. Graphs with more slots are sorted in
// parts of whole sources (k_wide_gather). DANCE_REVERSE_PART_ITEMS lowers the
// cap so that tests run the split path on small graphs; results are equal.
static size_t reverse_part_cap(uint32_t R) {
  size_t cap = 0xFFFFFFFFull;
  const char* e = std::getenv("DANCE_REVERSE_PART_ITEMS");
  if (e && e[0]) {
    const size_t v = (size_t)std::strtoull(e, nullptr, 10);
    if (v > 0 && v < cap) cap = v;
  }
  return std::max<size_t>(cap, std::max(R, 1u));
}
// Parts (1: one sort over every slot) and sources per part.
static void reverse_parts(uint32_t N, uint32_t R, uint32_t* parts, uint32_t* per) {
  const size_t items = (size_t)N * R, cap = reverse_part_cap(R);
  if (items <= cap) {
    *parts = 1;
    *per = N;
    return;
  }
  size_t np = (items + cap - 1) / cap;
  size_t ps = (N + np - 1) / np;
  while (ps * R > cap) {
    ++np;
    ps = (N + np - 1) / np;
  }
  *per = (uint32_t)ps;
  *parts = (uint32_t)((N + ps - 1) / ps);
}

struct ReverseWs {
  DevBuf keys[2], vals[2], offs, order, snap;
  SortWorkspace sort;
  ScanWorkspace scan;
  // split sort (graphs of 2^32 or more slots)
  uint32_t parts = 1, per = 0;
  DevBuf pvals, poffs, offs64, src_sorted, snap_sorted;
  int alloc(uint32_t N, uint32_t R) {
    const size_t items = (size_t)N * R;
    reverse_parts(N, R, &parts, &per);
    // the locality schedule sorts N items in these buffers first
    const size_t sort_items = std::max<size_t>(parts == 1 ? items : (size_t)per * R, std::max(N, 1u));
    for (int i = 0; i < 2; ++i) {
      DCHECK(keys[i].alloc(sort_items * 4));
      DCHECK(vals[i].alloc(sort_items * 4));
    }
    DCHECK(snap.alloc(std::max<size_t>(items, 1) * 4));
    DCHECK(offs.alloc(((size_t)N + 1) * 4));
    if (parts > 1) {
      DCHECK(pvals.alloc(items * 4));
      DCHECK(poffs.alloc((size_t)parts * ((size_t)N + 1) * 4));
      DCHECK(offs64.alloc(((size_t)N + 1) * 8));
      DCHECK(src_sorted.alloc(items * 4));
      DCHECK(snap_sorted.alloc(items * 4));
    }
    return 0;
  }
};

// The reverse CSR as the merge reads it (MergeArgs: offsets, srcs, snap,
// offsets64).
struct RevCsr {
  const uint32_t* offs;
  const uint32_t* srcs;
  const float* snap;
  const uint64_t* offs64;
};

// Reverse CSR in canonical (ascending source) order. One sort: srcs are the
// sorted forward slots (s*R + i) and snap their distances by slot. Split sort:
// srcs and snap hold each sorted position's source and distance, offs64 the
// 64-bit offsets.
static int build_reverse_csr(GraphBufs g, ReverseWs& ws, hipStream_t s, RevCsr* out) {
  const size_t items = (size_t)g.N * g.R;
  uint32_t* kb[2] = {ws.keys[0].as<uint32_t>(), ws.keys[1].as<uint32_t>()};
  uint32_t* vb[2] = {ws.vals[0].as<uint32_t>(), ws.vals[1].as<uint32_t>()};
  if (ws.parts == 1) {
    if (items > 0) {
      hipLaunchKernelGGL(k_rev_keys, dim3((uint32_t)((items + 255) / 256)), dim3(256), 0, s, g.work, g.deg_work,
                         g.wd, g.N, g.R, g.C, 0u, items, kb[0], vb[0], ws.snap.as<float>());
      DHIP(hipGetLastError());
    }
    int which = 0;
    DCHECK(radix_sort_pairs(kb, vb, items, bit_length(g.N), ws.sort, s, &which));
    hipLaunchKernelGGL(k_seg_offsets, dim3((uint32_t)((items + 1 + 255) / 256)), dim3(256), 0, s, kb[which], items,
                       g.N, ws.offs.as<uint32_t>());
    DHIP(hipGetLastError());
    *out = RevCsr{ws.offs.as<const uint32_t>(), vb[which], ws.snap.as<const float>(), nullptr};
    return 0;
  }
  if (ws.parts > kMaxRevParts) {
    std::fprintf(stderr, "[gpu_vamana_build] N*R=%zu needs %u reverse parts, above %u\n", items, ws.parts,
                 kMaxRevParts);
    return -1;
  }
  WideParts wp{};
  wp.P = ws.parts;
  size_t base = 0;
  for (uint32_t p = 0; p < ws.parts; ++p) {
    const uint32_t s_lo = p * ws.per, s_hi = std::min(g.N, s_lo + ws.per);
    const size_t items_p = (size_t)(s_hi - s_lo) * g.R;
    wp.s_lo[p] = s_lo;
    wp.vbase[p] = base;
    hipLaunchKernelGGL(k_rev_keys, dim3((uint32_t)((items_p + 255) / 256)), dim3(256), 0, s, g.work, g.deg_work,
                       g.wd, g.N, g.R, g.C, s_lo, items_p, kb[0], vb[0], ws.snap.as<float>());
    DHIP(hipGetLastError());
    int which = 0;
    DCHECK(radix_sort_pairs(kb, vb, items_p, bit_length(g.N), ws.sort, s, &which));
    hipLaunchKernelGGL(k_seg_offsets, dim3((uint32_t)((items_p + 1 + 255) / 256)), dim3(256), 0, s, kb[which],
                       items_p, g.N, ws.poffs.as<uint32_t>() + (size_t)p * ((size_t)g.N + 1));
    DHIP(hipGetLastError());
    DHIP(hipMemcpyAsync(ws.pvals.as<uint32_t>() + base, vb[which], items_p * 4, hipMemcpyDeviceToDevice, s));
    base += items_p;
  }
  hipLaunchKernelGGL(k_wide_offsets, dim3((g.N + 1 + 255) / 256), dim3(256), 0, s, g.N, wp,
                     ws.poffs.as<const uint32_t>(), ws.offs64.as<uint64_t>());
  DHIP(hipGetLastError());
  hipLaunchKernelGGL(k_wide_gather, grid_dims(((uint64_t)g.N + 3) / 4, 256), dim3(256), 0, s, g.N, g.R, wp, ws.poffs.as<const uint32_t>(),
                     ws.pvals.as<const uint32_t>(), ws.snap.as<const float>(), ws.offs64.as<const uint64_t>(),
                     ws.src_sorted.as<uint32_t>(), ws.snap_sorted.as<float>());
  DHIP(hipGetLastError());
  *out = RevCsr{nullptr, ws.src_sorted.as<const uint32_t>(), ws.snap_sorted.as<const float>(),
                ws.offs64.as<const uint64_t>()};
  return 0;
}

static int launch_merge(const Rows& rows, GraphBufs g, const RevCsr& rev, const Profile& prof, const uint32_t* order,
                        VCounters* ctr, hipStream_t s) {
  const int cpl = pick_cpl(rows.rs.nch);
  const uint32_t Cp = round64(g.C);
  MergeArgs a{rows.rs, g, rev.offs, rev.srcs, rev.snap, prof.heavy_threshold, prof.heavy_sample, order, ctr,
              rev.offs64};
  return with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
    constexpr int DT = decltype(dt)::value, CPL = decltype(c)::value;
    if (g.C <= 64)
      hipLaunchKernelGGL((k_merge_reg<DT, CPL, 1>), xcd_grid(g.N), dim3(kBlock), 0, s, a);
    else if (g.C <= 128)
      hipLaunchKernelGGL((k_merge_reg<DT, CPL, 2>), xcd_grid(g.N), dim3(kBlock), 0, s, a);
    else if (g.C <= 256)
      hipLaunchKernelGGL((k_merge_reg<DT, CPL, 4>), xcd_grid(g.N), dim3(kBlock), 0, s, a);
    else
      hipLaunchKernelGGL((k_merge<DT, CPL>), xcd_grid(g.N), dim3(kBlock),
                         (size_t)kWavesPerBlock * merge_lds_words(Cp) * 4, s, a, Cp);
    DHIP(hipGetLastError());
    return 0;
  });
}

// Iteration count (VAMANA_ITERS, gpu_vamana_config.h:78-79, a compile-time
// constant of the reference; the loop at vnew2.cu:2517-2637): the run-time
// setting DANCE_VAMANA_ITERS, 1..kMaxIters, default 4. The schedule follows
// the count: alpha in the last iteration, the fill to kFinalMinDegree in the
// last, the coarse STEPS cap in the first kCoarseIters. Returns 0 (no
// iteration) for a value outside the range.
static uint32_t vamana_iters() {
  const char* e = std::getenv("DANCE_VAMANA_ITERS");
  if (!(e && e[0])) return kDefaultIters;
  char* end = nullptr;
  const unsigned long v = std::strtoul(e, &end, 10);
  return (end && *end == '\0' && v >= 1 && v <= kMaxIters) ? (uint32_t)v : 0u;
}

// Alpha schedule (gpu_vamana_alpha_for_iter, vnew2.cu:201-213): iterations
// from DANCE_ALPHA_FROM_ITER on prune with alpha, earlier ones with 1. The
// default is the reference's (the last iteration only); 0 is its
// USE_ALPHA_FROM_FIRST_ITER=1 and k its VAMANA_ALPHA_FINAL_FROM_ITER=k.
static uint32_t alpha_from_iter(uint32_t iters) {
  const char* e = std::getenv("DANCE_ALPHA_FROM_ITER");
  if (e && e[0]) return (uint32_t)std::strtoul(e, nullptr, 10);
  return iters - 1;
}

// Locality schedule (see k_cells_q / k_cells): order[] = vertices sorted by
// their nearest pivots. Pivots are K evenly spaced rows. K comes from
// DANCE_LOCALITY_CELLS (0 disables the schedule), by default 1024 for float
// rows and 1536 for uint8 rows, the fastest counts with three-pivot keys
// (c3 3.588 s at 1024 against 3.596 at 1536 and 3.594 / 3.630 at 512 / 256;
// c4 2.525 s at 1024 against 2.516 at 1536 and 2.539 at 1625). Uses the
// reverse-sort buffers as scratch.
static uint32_t locality_cells(int dtype) {
  const char* e = std::getenv("DANCE_LOCALITY_CELLS");
  if (e && e[0]) return (uint32_t)std::strtoul(e, nullptr, 10);
  return dtype == DANCE_U8 ? 1536u : 1024u;
}


static int build_schedule(const Rows& rows, const QBoundSet& qb, ReverseWs& ws, hipStream_t s,
                          const uint32_t** order_out) {
  const uint32_t N = rows.N;
  const uint32_t K = std::min(locality_cells(rows.dtype), N);
  *order_out = nullptr;
  if (K < 2) return 0;
  DevBuf dpiv;
  DCHECK(dpiv.alloc(K * 4));
  hipLaunchKernelGGL(k_pivots, dim3((K + 255) / 256), dim3(256), 0, s, N, K, dpiv.as<uint32_t>());
  DHIP(hipGetLastError());
  const int cpl = pick_cpl(rows.rs.nch);
  uint32_t* kb[2] = {ws.keys[0].as<uint32_t>(), ws.keys[1].as<uint32_t>()};
  uint32_t* vb[2] = {ws.vals[0].as<uint32_t>(), ws.vals[1].as<uint32_t>()};
  // Vertices sorted by their three nearest pivots (cell, then the cells it
  // faces): c4 2.63 -> 2.57 s and c3 3.697 -> 3.689 s against the cell alone,
  // same graphs.
  const uint32_t lv = cell_levels(K, 3);
  // the same cells from int8 MFMA tiles (DANCE_CELLS_MFMA=0: the dot-product
  // kernel k_cells_q); one wave per 32 vertices
  const char* em = std::getenv("DANCE_CELLS_MFMA");
  const bool mfma_cells = !(em && em[0] == '0');
  const dim3 mgrid((uint32_t)(((uint64_t)N + 127) / 128));
  if (qb.rows && mfma_cells) {
    hipLaunchKernelGGL(k_cells_mfma<false>, mgrid, dim3(256), 0, s, qb.rows, kQChunks, N, dpiv.as<uint32_t>(), K,
                       lv, kb[0], vb[0]);
    DHIP(hipGetLastError());
  } else if (qb.rows) {
    // integer-code pivot search on the quantized rows
    hipLaunchKernelGGL(k_cells_q<false>, dim3((N + 255) / 256), dim3(256), 0, s, qb.rows, kQChunks, kQChunks, N,
                       dpiv.as<uint32_t>(), K, lv, kb[0], vb[0]);
    DHIP(hipGetLastError());
  } else if (rows.dtype == DANCE_U8 && rows.rs.stride16 == 8u && mfma_cells) {  // 128-byte rows
    hipLaunchKernelGGL(k_cells_mfma<true>, mgrid, dim3(256), 0, s, rows.rs.rows, rows.rs.stride16, N,
                       dpiv.as<uint32_t>(), K, lv, kb[0], vb[0]);
    DHIP(hipGetLastError());
  } else if (rows.dtype == DANCE_U8 && rows.rs.nch <= 8) {
    hipLaunchKernelGGL(k_cells_q<true>, dim3((N + 255) / 256), dim3(256), 0, s, rows.rs.rows, rows.rs.stride16,
                       rows.rs.nch, N, dpiv.as<uint32_t>(), K, lv, kb[0], vb[0]);
    DHIP(hipGetLastError());
  } else {
    DCHECK(with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
      hipLaunchKernelGGL((k_cells<decltype(dt)::value, decltype(c)::value>), dim3(cells_grid(N)),
                         dim3(kCellsBlock), 0, s, rows.rs, N, dpiv.as<uint32_t>(), K, lv, kb[0], vb[0]);
      DHIP(hipGetLastError());
      return 0;
    }));
  }
  int which = 0;
  const uint64_t nkeys = lv == 3u ? (uint64_t)K * K * K : (uint64_t)K;
  DCHECK(radix_sort_pairs(kb, vb, N, bit_length((uint32_t)(nkeys - 1)), ws.sort, s, &which));
  // Keep the order in the offsets-sized scratch that is free until the first
  // reverse step: copy into its own buffer owned by the workspace.
  DCHECK(ws.order.alloc((size_t)N * 4));
  DHIP(hipMemcpyAsync(ws.order.p, vb[which], (size_t)N * 4, hipMemcpyDeviceToDevice, s));
  DHIP(hipStreamSynchronize(s));
  *order_out = ws.order.as<uint32_t>();
  return 0;
}

// ---------------------------------------------------------------------------
// Full build on resident rows.
// ---------------------------------------------------------------------------
// Stage timing events. With `on` false (the allocation-free entry) no event is
// created: make() returns null, record() does nothing and the stage times
// read 0.
struct StageEvents {
  bool on = true;
  std::vector<hipEvent_t> ev;
  ~StageEvents() {
    for (auto e : ev) (void)hipEventDestroy(e);
  }
  int make(hipEvent_t* e) {
    *e = nullptr;
    if (!on) return 0;
    DHIP(hipEventCreate(e));
    ev.push_back(*e);
    return 0;
  }
};

static int record(hipEvent_t e, hipStream_t s) {
  if (e) DHIP(hipEventRecord(e, s));
  return 0;
}

static float elapsed_ms(hipEvent_t a, hipEvent_t b) {
  float ms = 0.f;
  if (a && b && hipEventElapsedTime(&ms, a, b) == hipSuccess) return ms;
  return 0.f;
}

// Rows wider than the widest compiled chunk group (16 chunks of 16 bytes per
// lane of an octet) are rejected before any device call.
static int check_width(uint32_t dim, int store) {
  if (pick_cpl((uint32_t)(((uint64_t)dim * elem_bytes(store) + 15) / 16)) < 0) {
    std::fprintf(stderr, "[gpu_vamana_build] dim=%u is beyond the supported row width\n", dim);
    return -1;
  }
  return 0;
}

static int validate(uint32_t N, uint32_t dim, uint32_t R, uint32_t L, uint32_t C, uint32_t& STEPS) {
  if (N == 0 || dim == 0 || R == 0 || L == 0 || C == 0 || STEPS == 0) {
    std::fprintf(stderr, "[gpu_vamana_build] invalid parameters: N=%u dim=%u R=%u L=%u C=%u STEPS=%u\n", N, dim, R, L,
                 C, STEPS);
    return -1;
  }
  if (C < R) {
    std::fprintf(stderr, "[gpu_vamana_build] invalid parameters: C=%u must be >= R=%u\n", C, R);
    return -1;
  }
  if (STEPS > L) {
    std::fprintf(stderr, "[gpu_vamana_build] STEPS=%u is larger than L=%u, clamp STEPS to L.\n", STEPS, L);
    STEPS = L;
  }
  if (L > kMaxBuildL) {
    std::fprintf(stderr, "[gpu_vamana_build] L=%u exceeds the supported maximum %u\n", L, kMaxBuildL);
    return -1;
  }
  if (vamana_iters() == 0) {
    std::fprintf(stderr, "[gpu_vamana_build] DANCE_VAMANA_ITERS=%s is not an iteration count in 1..%u\n",
                 std::getenv("DANCE_VAMANA_ITERS"), kMaxIters);
    return -1;
  }
  uint32_t parts = 1, per = 0;
  reverse_parts(N, R, &parts, &per);
  if (parts > kMaxRevParts) {
    std::fprintf(stderr, "[gpu_vamana_build] N*R=%llu exceeds %u reverse-sort parts of 2^32 - 1 slots\n",
                 (unsigned long long)N * R, kMaxRevParts);
    return -1;
  }
  return 0;
}

// Runs the whole build. On success st.cur/deg_cur hold the graph.
// Callers hold g_mu and pass the active profile.
static int run_build(const Rows& rows, uint32_t R, uint32_t L, uint32_t C, uint32_t STEPS, const Profile& prof,
                     State& st, hipStream_t s, GPUVamanaStats* stats, DanceKernelProfile* kp, uint32_t* medoid_out,
                     bool timed = true) {
  const uint32_t N = rows.N;
  if (pick_cpl(rows.rs.nch) < 0) {
    std::fprintf(stderr, "[gpu_vamana_build] dim=%u is beyond the supported row width\n", rows.dim);
    return -1;
  }
  DCHECK(st.alloc(N, R, C, st.cur.p == nullptr, st.deg_cur.p == nullptr));
  ReverseWs rws;
  DCHECK(rws.alloc(N, R));
  DevBuf ctr_buf, csum, scores, cands;
  DCHECK(ctr_buf.alloc(sizeof(VCounters) * kCtrStripes));
  DCHECK(csum.alloc(sizeof(VCounters)));
  DHIP(hipMemsetAsync(ctr_buf.p, 0, sizeof(VCounters) * kCtrStripes, s));
  VCounters* ctr = ctr_buf.as<VCounters>();
  GraphBufs g = st.g();
  StageEvents E;
  E.on = timed;
  hipEvent_t e0, e_med, e_init;
  DCHECK(E.make(&e0));
  DCHECK(E.make(&e_med));
  DCHECK(E.make(&e_init));
  DCHECK(record(e0, s));

  // Approximate medoid (vnew2.cu:2359-2479): device scores, host top-1.
  const double t_med = now_sec();
  const uint32_t nc = std::min(kMedoidCandidates, N), ns = std::min(kMedoidSamples, N);
  DCHECK(scores.alloc(nc * 4));
  DCHECK(cands.alloc(nc * 4));
  DCHECK(launch_medoid(rows, s, scores.as<float>(), cands.as<uint32_t>(), nc, ns));
  float hs[kMedoidCandidates];
  uint32_t hc[kMedoidCandidates];
  DHIP(hipMemcpyAsync(hs, scores.p, nc * 4, hipMemcpyDeviceToHost, s));
  DHIP(hipMemcpyAsync(hc, cands.p, nc * 4, hipMemcpyDeviceToHost, s));
  DCHECK(record(e_med, s));
  DHIP(hipStreamSynchronize(s));
  uint32_t best = DANCE_INV;
  float bs = FLT_MAX;
  for (uint32_t i = 0; i < nc; ++i)
    if (hs[i] < bs) {
      bs = hs[i];
      best = i;
    }
  const uint32_t start = best == DANCE_INV ? 0u : hc[best];
  if (stats) stats->medoid_seconds = now_sec() - t_med;

  // At L <= 128 the first search launch computes the initial rows itself
  // (its hashed-neighbour variants), and nothing reads cur, work or wd
  // before it; k_init runs for the other variants only.
  const bool init_in_search = L <= 128;
  if (!init_in_search) DCHECK(launch_init(rows, g, s));
  DevBuf qbuf;
  QBoundSet qb{};
  DCHECK(build_qbound(rows, qbuf, s, &qb));
  const uint32_t* order = nullptr;
  DCHECK(build_schedule(rows, qb, rws, s, &order));
  uint32_t q_iters = qbound_iters();  // the last iteration's bit may be set after the one before it
  const uint32_t ib_iters = insert_bound_iters();
  uint32_t q_prune_iters = qbound_prune_iters();  // iteration 1's bit may be set after iteration 0
  const uint32_t iters = vamana_iters();
  if (iters == 0) return -1;  // validate() reports it
  const uint32_t a_from = alpha_from_iter(iters);
  const uint32_t p_rank = prune_rank_iters(rows.dtype);
  DCHECK(record(e_init, s));

  VCounters before_last{};  // cumulative counters after iteration iters - 3 (zero if none)
  DevBuf snaps;  // timed builds: iters cumulative counter snapshots
  if (timed) DCHECK(snaps.alloc(sizeof(VCounters) * kMaxIters));
  struct IterEv {
    hipEvent_t s0, s1, r1, m1, p1;
  };
  IterEv iev[kMaxIters];
  for (auto& ie : iev) {
    DCHECK(E.make(&ie.s0));
    DCHECK(E.make(&ie.s1));
    DCHECK(E.make(&ie.r1));
    DCHECK(E.make(&ie.m1));
    DCHECK(E.make(&ie.p1));
  }
  for (uint32_t it = 0; it < iters; ++it) {
    const float alpha = it >= a_from ? kAlpha : 1.0f;
    uint32_t steps = STEPS;
    if (it < kCoarseIters && steps > kWarmupSteps) steps = kWarmupSteps;
    if (verbose())
      std::printf("[gpu_vamana_build] iteration %u / %u, alpha=%.3f\n", it + 1, iters, (double)alpha);
    DCHECK(record(iev[it].s0, s));
    const QBoundSet qb_it = ((q_iters >> it) & 1u) ? qb : QBoundSet{nullptr, 0.0f, 0.0f};
    DCHECK(launch_search(rows, g, L, steps, alpha, start, order, ctr, qb_it, s, ((ib_iters >> it) & 1u) != 0,
                         it == 0));  // k_init wrote cur just before
    DCHECK(record(iev[it].s1, s));
    RevCsr rev{};
    DCHECK(build_reverse_csr(g, rws, s, &rev));
    DCHECK(record(iev[it].r1, s));
    DCHECK(launch_merge(rows, g, rev, prof, order, ctr, s));
    DCHECK(record(iev[it].m1, s));
    const uint32_t md = (it + 1 == iters) ? kFinalMinDegree : 0u;
    const QBoundSet qp_it = ((q_prune_iters >> it) & 1u) ? qb : QBoundSet{nullptr, 0.0f, 0.0f};
    DCHECK(launch_prune(rows, g, md, alpha, order, ctr, qp_it, ((p_rank >> it) & 1u) != 0u, s));
    DCHECK(record(iev[it].p1, s));
    if (it == 0 && qb.rows && qbound_prune_adaptive() && !((q_prune_iters >> 1) & 1u) && iters > 1) {
      // pair density of iteration 0's prune (its bound checks), read once
      hipLaunchKernelGGL(k_ctr_sum, dim3(1), dim3(64), 0, s, static_cast<const VCounters*>(ctr),
                         csum.as<VCounters>());
      DHIP(hipGetLastError());
      VCounters h{};
      DHIP(hipMemcpyAsync(&h, csum.p, sizeof(VCounters), hipMemcpyDeviceToHost, s));
      DHIP(hipStreamSynchronize(s));
      const double pairs = (double)g.C * (double)(g.C > 0 ? g.C - 1 : 0) / 8.0;
      if ((double)h.prune_bound_checks > pairs * (double)g.N) q_prune_iters |= 2u;
    }
    if (qb.rows && qbound_iters_adaptive() && iters > 1 && it + 3 >= iters && it + 1 < iters) {
      // candidate distances per expansion of the iteration before the last:
      // cumulative counters after iterations iters - 3 and iters - 2
      hipLaunchKernelGGL(k_ctr_sum, dim3(1), dim3(64), 0, s, static_cast<const VCounters*>(ctr),
                         csum.as<VCounters>());
      DHIP(hipGetLastError());
      VCounters h{};
      DHIP(hipMemcpyAsync(&h, csum.p, sizeof(VCounters), hipMemcpyDeviceToHost, s));
      DHIP(hipStreamSynchronize(s));
      if (it + 3 == iters) {
        before_last = h;
      } else {
        const double cand = (double)(h.search_dist + h.bound_skips) -
                            (double)(before_last.search_dist + before_last.bound_skips);
        const double exps = (double)(h.expansions - before_last.expansions);
        if (cand > kQBoundLastMinDist * exps) q_iters |= 1u << (iters - 1);
      }
    }
    if (timed) {  // cumulative counters after this iteration
      hipLaunchKernelGGL(k_ctr_sum, dim3(1), dim3(64), 0, s, static_cast<const VCounters*>(ctr),
                         snaps.as<VCounters>() + it);
      DHIP(hipGetLastError());
    }
  }
  DHIP(hipStreamSynchronize(s));
  DHIP(hipGetLastError());

  VCounters hc_ctr{};
  {
    VCounters stripes[kCtrStripes];
    DHIP(hipMemcpyAsync(stripes, ctr_buf.p, sizeof(VCounters) * kCtrStripes, hipMemcpyDeviceToHost, s));
    DHIP(hipStreamSynchronize(s));
    static_assert(sizeof(VCounters) % sizeof(unsigned long long) == 0, "VCounters holds u64 fields only");
    const size_t nf = sizeof(VCounters) / sizeof(unsigned long long);
    auto* dst = reinterpret_cast<unsigned long long*>(&hc_ctr);
    for (const VCounters& st : stripes) {
      const auto* src = reinterpret_cast<const unsigned long long*>(&st);
      for (size_t f = 0; f < nf; ++f) dst[f] += src[f];
    }
  }
  VCounters hsnap[kMaxIters] = {};
  if (timed) {
    DHIP(hipMemcpyAsync(hsnap, snaps.p, sizeof(VCounters) * iters, hipMemcpyDeviceToHost, s));
    DHIP(hipStreamSynchronize(s));
  }
  DanceKernelProfile p{};
  p.iterations = iters;
  p.vector_bytes = rows.vbytes();
  p.medoid_ms = elapsed_ms(e0, e_med);
  p.init_ms = elapsed_ms(e_med, e_init);
  for (uint32_t it = 0; it < iters; ++it) {
    p.search_iter_ms[it] = elapsed_ms(iev[it].s0, iev[it].s1);
    p.prune_iter_ms[it] = elapsed_ms(iev[it].m1, iev[it].p1);
    p.search_ms += p.search_iter_ms[it];
    p.reverse_ms += elapsed_ms(iev[it].s1, iev[it].r1);
    p.merge_ms += elapsed_ms(iev[it].r1, iev[it].m1);
    p.prune_ms += p.prune_iter_ms[it];
  }
  p.total_ms = elapsed_ms(e0, iev[iters - 1].p1);
  p.search_dist = hc_ctr.search_dist;
  p.insert_dist = hc_ctr.insert_dist;
  p.expansions = hc_ctr.expansions;
  p.vis_skips = hc_ctr.vis_skips;
  p.merge_dist = hc_ctr.merge_dist;
  p.prune_dist = hc_ctr.prune_dist;
  p.reverse_edges = hc_ctr.reverse_edges;
  p.touched_rows = hc_ctr.touched_rows;
  p.cyc_select = hc_ctr.cyc_select;
  p.cyc_insert = hc_ctr.cyc_insert;
  p.cyc_dist = hc_ctr.cyc_dist;
  p.cyc_pool = hc_ctr.cyc_pool;
  p.cyc_seed = hc_ctr.cyc_seed;
  p.cyc_total = hc_ctr.cyc_total;
  p.bound_checks = hc_ctr.bound_checks;
  p.bound_skips = hc_ctr.bound_skips;
  p.prune_bound_checks = hc_ctr.prune_bound_checks;
  p.prune_bound_skips = hc_ctr.prune_bound_skips;
  p.prune_rounds = hc_ctr.prune_rounds;
  p.prune_exact_rounds = hc_ctr.prune_exact_rounds;
  p.cyc_prune_rank = hc_ctr.cyc_prune_rank;
  p.cyc_prune_gram = hc_ctr.cyc_prune_gram;
  p.cyc_prune_rounds = hc_ctr.cyc_prune_rounds;
  p.cyc_prune_fill = hc_ctr.cyc_prune_fill;
  p.insert_bound_checks = hc_ctr.insert_bound_checks;
  p.insert_bound_skips = hc_ctr.insert_bound_skips;
  const double V = rows.vbytes();
  for (uint32_t it = 0; timed && it < iters; ++it) {
    const VCounters& c = hsnap[it];
    const VCounters z{};
    const VCounters& b = it ? hsnap[it - 1] : z;
    p.search_dist_iter[it] = c.search_dist - b.search_dist;
    p.insert_dist_iter[it] = c.insert_dist - b.insert_dist;
    p.expansions_iter[it] = c.expansions - b.expansions;
    p.bound_checks_iter[it] = c.bound_checks - b.bound_checks;
    p.bound_skips_iter[it] = c.bound_skips - b.bound_skips;
    p.merge_dist_iter[it] = c.merge_dist - b.merge_dist;
    p.prune_dist_iter[it] = c.prune_dist - b.prune_dist;
    p.prune_bound_checks_iter[it] = c.prune_bound_checks - b.prune_bound_checks;
    p.prune_bound_skips_iter[it] = c.prune_bound_skips - b.prune_bound_skips;
    p.insert_bound_checks_iter[it] = c.insert_bound_checks - b.insert_bound_checks;
    p.insert_bound_skips_iter[it] = c.insert_bound_skips - b.insert_bound_skips;
    // The first iteration's L <= 128 variants compute the random initial graph:
    // no adjacency or cur row is read, and each vertex gathers its R initial
    // neighbours' rows and writes its work row (8C) instead of reading and
    // writing it (16C).
    const bool init_it = it == 0 && L <= 128;
    const double adj = init_it ? 0.0 : 4.0 * R + 4.0;
    const double per_vertex = init_it ? V + R * V + 8.0 * C : V + 4.0 * R + 4.0 + 16.0 * C;
    p.search_bytes_iter[it] = (double)(p.search_dist_iter[it] + p.insert_dist_iter[it]) * V +
                              (double)p.expansions_iter[it] * adj + (double)N * per_vertex +
                              (double)(p.bound_checks_iter[it] + p.insert_bound_checks_iter[it]) * (kQChunks * 16.0);
    // the rank kernel with the bound reads every candidate's code row once;
    // k_prune reads the code rows of the pairs it tests; the rank kernel's
    // Gram tiles (uint8 rows) read every candidate's row once for all pairs
    const bool q_it = qb.rows && ((q_prune_iters >> it) & 1u);
    const bool rank_it = ((p_rank >> it) & 1u) && C <= kRankCap;
    const bool gram_it = rank_it && rows.dtype == DANCE_U8 && prune_gram();
    const double qbytes = !q_it ? 0.0
                          : rank_it ? (double)N * C * (kQChunks * 16.0)
                                    : (double)p.prune_bound_checks_iter[it] * (kQChunks * 16.0);
    const double pair_rows = gram_it ? (double)N * C : (double)p.prune_dist_iter[it];
    p.prune_bytes_iter[it] = pair_rows * V + (double)N * (24.0 * C) + qbytes;
  }
  p.search_bytes = (double)(p.search_dist + p.insert_dist) * V + (double)p.expansions * (4.0 * R + 4.0) +
                   (double)iters * N * (V + 4.0 * R + 4.0 + 16.0 * C) +
                   (double)(p.bound_checks + p.insert_bound_checks) * (kQChunks * 16.0);
  if (timed) {  // the per-launch figures know which launch recomputed its adjacency rows
    p.search_bytes = 0.0;
    for (uint32_t it = 0; it < iters; ++it) p.search_bytes += p.search_bytes_iter[it];
  }
  p.merge_bytes = (double)p.merge_dist * 4.0 + (double)p.reverse_edges * 4.0 +
                  (double)p.touched_rows * (16.0 * C + 8.0);
  p.prune_bytes = (double)p.prune_dist * V + (double)iters * N * (24.0 * C) +
                  (double)p.prune_bound_checks * (kQChunks * 16.0);
  if (timed) {  // the per-launch figures know which launches used Gram tiles
    p.prune_bytes = 0.0;
    for (uint32_t it = 0; it < iters; ++it) p.prune_bytes += p.prune_bytes_iter[it];
  }
  const double items = (double)N * R;
  const double passes = (bit_length(N) + 7) / 8;
  p.reverse_bytes = (double)iters * (items * 16.0 + passes * items * 20.0);
  if (kp) *kp = p;
  if (stats) {
    stats->search_online_insert_seconds = p.search_ms * 1e-3;
    stats->reverse_seconds = (p.reverse_ms + p.merge_ms) * 1e-3;
    stats->reverse_csr_seconds = p.reverse_ms * 1e-3;
    stats->final_prune_seconds = p.prune_ms * 1e-3;
    stats->distance_computations = p.search_dist + p.insert_dist + p.prune_dist;
    stats->online_insert_attempts = hc_ctr.insert_try;
    stats->online_insert_mutations = hc_ctr.insert_mut;
    stats->reverse_proposals = p.reverse_edges;
    stats->reverse_touched_rows = p.touched_rows;
  }
  if (medoid_out) *medoid_out = start;
  if (verbose())
    std::printf("[gpu_vamana_build] N=%u dim=%u R=%u L=%u C=%u STEPS=%u profile=%s medoid=%u total=%.3f ms\n", N,
                rows.dim, R, L, C, STEPS, prof.name, start, p.total_ms);
  return 0;
}

template <typename HostT>
static int build_host(const HostT* h_data, int src_dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t L,
                      uint32_t C, uint32_t STEPS, uint32_t* h_graph, uint32_t* h_degree, void** keep_data,
                      uint32_t** keep_graph, uint32_t** keep_degree, Builder builder = Builder::vnew2) {
  std::lock_guard<std::mutex> lk(g_mu);
  (builder == Builder::v8 ? g_last_stats_v8 : g_last_stats) = GPUVamanaStats{};
  const double t0 = now_sec();
  const bool handoff = keep_data != nullptr;
  if (h_data == nullptr || (!handoff && (h_graph == nullptr || h_degree == nullptr))) {
    std::fprintf(stderr, "[gpu_vamana_build] null input pointer.\n");
    return -1;
  }
  DCHECK(validate(N, dim, R, L, C, STEPS));
  const Profile prof = profile_for(builder);
  const int store = (src_dtype == DANCE_F32 && prof.fp16) ? DANCE_F16 : src_dtype;
  if (builder == Builder::v8 && verbose())
    std::printf("[gpu_vamana_build] type=%s N=%u dim=%u R=%u L=%u C=%u STEPS=%u alpha=%.3f iters=%u builder=v8 "
                "profile=%s fp16=%u heavy_cap=0\n",
                store == DANCE_F16 ? "float16" : (src_dtype == DANCE_U8 ? "uint8" : "float"), N, dim, R, L,
                C, std::min(STEPS, L), (double)kAlpha, vamana_iters(), prof.name, prof.fp16 ? 1u : 0u);
  DCHECK(check_width(dim, store));
  hipStream_t s = nullptr;
  DHIP(hipStreamCreate(&s));
  struct StreamGuard {
    hipStream_t s;
    ~StreamGuard() {
      if (s) (void)hipStreamDestroy(s);
    }
  } sg{s};
  GPUVamanaStats stats{};
  const double th = now_sec();
  Rows rows;
  DevBuf handoff_data;
  if (handoff) {
    // The hand-off returns the caller-typed vectors (N x dim) in device memory.
    DCHECK(handoff_data.alloc((size_t)N * dim * sizeof(HostT)));
    DHIP(hipMemcpyAsync(handoff_data.p, h_data, (size_t)N * dim * sizeof(HostT), hipMemcpyHostToDevice, s));
    DCHECK(setup_rows(rows, handoff_data.p, true, src_dtype, store, N, dim, s));
  } else {
    DCHECK(setup_rows(rows, h_data, false, src_dtype, store, N, dim, s));
  }
  DHIP(hipStreamSynchronize(s));
  stats.h2d_seconds = now_sec() - th;
  State st;
  uint32_t medoid = 0;
  DanceKernelProfile kp{};
  DCHECK(run_build(rows, R, L, C, STEPS, prof, st, s, &stats, &kp, &medoid));
  const double td = now_sec();
  if (handoff) {
    *keep_data = handoff_data.release();
    *keep_graph = st.cur.as<uint32_t>();
    st.cur.release();
    *keep_degree = st.deg_cur.as<uint32_t>();
    st.deg_cur.release();
  } else {
    DHIP(hipStreamSynchronize(s));  // the staged copies run on streams of their own
    DCHECK(copy_pageable(h_graph, st.cur.p, (size_t)N * R * 4, hipMemcpyDeviceToHost));
    DCHECK(copy_pageable(h_degree, st.deg_cur.p, (size_t)N * 4, hipMemcpyDeviceToHost));
  }
  stats.d2h_seconds = now_sec() - td;
  stats.gpu_build_seconds = now_sec() - t0;
  if (builder == Builder::v8) {
    g_last_stats_v8 = stats;
    g_last_medoid_v8 = medoid;
  } else {
    g_last_stats = stats;
    g_last_medoid = medoid;
  }
  g_last_prof = kp;
  return 0;
}

// ---------------------------------------------------------------------------
// Stage hooks: upload host state, run one production kernel, download.
// ---------------------------------------------------------------------------
struct StageCtx {
  hipStream_t s = nullptr;
  Rows rows;
  State st;
  ~StageCtx() {
    if (s) (void)hipStreamDestroy(s);
  }
  int open(const void* h_data, int dtype, uint32_t N, uint32_t dim) {
    DHIP(hipStreamCreate(&s));
    return setup_rows(rows, h_data, false, dtype, dtype, N, dim, s);
  }
};

static int up(void* d, const void* h, size_t b, hipStream_t s) {
  if (b) DHIP(hipMemcpyAsync(d, h, b, hipMemcpyHostToDevice, s));
  return 0;
}
static int down(void* h, const void* d, size_t b, hipStream_t s) {
  if (b) DHIP(hipMemcpyAsync(h, d, b, hipMemcpyDeviceToHost, s));
  return 0;
}

static int upload_state(State& st, uint32_t N, uint32_t R, uint32_t C, const uint32_t* cur, const uint32_t* deg_cur,
                        const uint32_t* work, const uint32_t* deg_work, const float* wd, hipStream_t s) {
  DCHECK(st.alloc(N, R, C));
  if (cur) DCHECK(up(st.cur.p, cur, (size_t)N * R * 4, s));
  if (deg_cur) DCHECK(up(st.deg_cur.p, deg_cur, (size_t)N * 4, s));
  DCHECK(up(st.work.p, work, (size_t)N * C * 4, s));
  DCHECK(up(st.deg_work.p, deg_work, (size_t)N * 4, s));
  DCHECK(up(st.wd.p, wd, (size_t)N * C * 4, s));
  return 0;
}

static int download_state(State& st, uint32_t* cur, uint32_t* deg_cur, uint32_t* work, uint32_t* deg_work, float* wd,
                          hipStream_t s) {
  const size_t N = st.N, R = st.R, C = st.C;
  if (cur) DCHECK(down(cur, st.cur.p, N * R * 4, s));
  if (deg_cur) DCHECK(down(deg_cur, st.deg_cur.p, N * 4, s));
  if (work) DCHECK(down(work, st.work.p, N * C * 4, s));
  if (deg_work) DCHECK(down(deg_work, st.deg_work.p, N * 4, s));
  if (wd) DCHECK(down(wd, st.wd.p, N * C * 4, s));
  DHIP(hipStreamSynchronize(s));
  return 0;
}

// Pairwise canonical distances: one wave per 64 pairs through batch_dist.
template <int DT, int CPL>
__global__ __launch_bounds__(kBlock) void k_pair_dist(RowSet rs, const uint32_t* __restrict__ a,
                                                      const uint32_t* __restrict__ b, uint64_t n,
                                                      float* __restrict__ out) {
  const uint32_t w = wave_index();
  const uint64_t base = ((uint64_t)blockIdx.x * kWavesPerBlock + w) * 64;
  if (base >= n) return;
  const uint32_t lane = lane_id(), grp = lane >> 3, sub = lane & 7u;
  for (uint32_t p = 0; p < 64; p += 8) {
    const uint64_t k = base + p + grp;
    const bool act = k < n;
    uint4 va[CPL], vb[CPL];
    load_row<CPL>(rs, act ? a[k] : 0u, act, sub, va);
    load_row<CPL>(rs, act ? b[k] : 0u, act, sub, vb);
    const float d = octet_finish<DT, CPL>(rs, sub, va, vb);
    if (act && sub == 0) out[k] = d;
  }
}

// The search's bound test on explicit pairs: flag[k] = 1 when the quantized
// bound proves dist(a[k], b[k]) >= T[k] (the querying row is a[k]).
__global__ __launch_bounds__(kBlock) void k_qbound_pairs(QBoundSet qb, const uint32_t* __restrict__ a,
                                                         const uint32_t* __restrict__ b,
                                                         const float* __restrict__ T, uint64_t n,
                                                         uint32_t* __restrict__ flag) {
  const uint32_t w = wave_index();
  const uint64_t base = ((uint64_t)blockIdx.x * kWavesPerBlock + w) * 64;
  if (base >= n) return;
  const uint32_t lane = lane_id(), grp = lane >> 3, sub = lane & 7u;
  for (uint32_t p = 0; p < 64; p += 8) {
    const uint64_t k = base + p + grp;
    const bool act = k < n;
    // the querying row differs per octet here, so its header is read per lane
    const uint4* qa = qb.rows + (size_t)(act ? a[k] : 0u) * kQChunks;
    const uint4 h = qa[0];
    const QSelf me{qa, __uint_as_float(h.x), __uint_as_float(h.y), __uint_as_float(h.z)};
    const float t = ((act ? T[k] : 0.0f) + qb.eta) * (1.0f + qb.kappa2);
    const float sT = (__builtin_sqrtf(t) + me.r) * (1.0f + kQSlack);
    const uint4 code = qa[sub];
    const uint4 bc = q_load(qb, act ? b[k] : 0u, act, sub);
    const bool rej = q_proves_reject(me, code, sT, bc, act, sub);
    if (act && sub == 0) flag[k] = rej ? 1u : 0u;
  }
}

// The online insert's occlusion-pair bounds on explicit pairs, as
// occlusion_bounded evaluates them (x = a[k], y = b[k], T0 = d_px):
// out[k] = 1 when the upper bound proves fl(alpha * dist) <= T0[k], 2 when
// the lower bound proves fl(alpha * dist) > T0[k], 0 when the pair is open.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_insert_bound_pairs(QBoundSet qb, const uint32_t* __restrict__ a,
                                                               const uint32_t* __restrict__ b,
                                                               const float* __restrict__ T0, float alpha, uint64_t n,
                                                               uint32_t* __restrict__ out) {
  const uint32_t w = wave_index();
  const uint64_t base = ((uint64_t)blockIdx.x * kWavesPerBlock + w) * 64;
  if (base >= n) return;
  const uint32_t lane = lane_id(), grp = lane >> 3, sub = lane & 7u;
  for (uint32_t p = 0; p < 64; p += 8) {
    const uint64_t k = base + p + grp;
    const bool act = k < n;
    // x differs per octet here, so its header is read per lane
    const uint4* qx = qb.rows + (size_t)(act ? a[k] : 0u) * kQChunks;
    const uint4 h = qx[0];
    const float xs = __uint_as_float(h.x), xr = __uint_as_float(h.y), xa = __uint_as_float(h.z);
    const float t0 = act ? T0[k] : 0.0f;
    const float ub = q_ub_root_of<DT>(qb, t0, alpha);
    const float lbT = (prune_bound_root(qb, t0, alpha) + xr) * (1.0f + kQSlack);
    const uint4 xcode = qx[sub];
    const uint4 bc = q_load(qb, act ? b[k] : 0u, act, sub);
    const int c = q_octet_dot(xcode, bc, sub);
    const float sy = __uint_as_float(bc.x), ry = __uint_as_float(bc.y), ay = __uint_as_float(bc.z);
    const bool yes = q_pair_ub(xs, xa, xr, ub, sy, ry, ay, c);
    const bool no = q_pair_proves(xs, xa, lbT, sy, ry, ay, c);
    if (act && sub == 0) out[k] = yes ? 1u : (no ? 2u : 0u);
  }
}

}  // namespace dance

using namespace dance;

// ===========================================================================
// Reference ABI
// ===========================================================================
// ---------------------------------------------------------------------------
// Device-resident build, and its allocation-free form.
// ---------------------------------------------------------------------------

// Scratch of the allocation-free build: one array per GPU, held until the
// process ends. Host code never passes `scratch` itself to the device (the
// name is a host-side stand-in); it uses the address hipGetSymbolAddress
// returns on each device (scratch_base). Calls of the allocation-free entry
// share that array; the library lock serialises them within a process.
constexpr size_t kScratchBytes = 256ull << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];

// Device address of this GPU's scratch array (looked up once per device, with
// that device current). Callers hold g_mu.
static int scratch_base(void** out) {
  int dev = 0;
  DHIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) {
    std::fprintf(stderr, "[gpu_vamana_build] device %d is beyond the scratch table\n", dev);
    return -1;
  }
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    DHIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

// Upper bound of the device bytes a resident build takes from the arena: the
// same buffers run_build, setup_rows and the radix sort allocate, each rounded
// up to the arena's 256-byte alignment.
static size_t resident_build_bytes(const void* d_data, int dtype, int store, uint32_t N, uint32_t dim, uint32_t R,
                                   uint32_t C, bool rows_ready = false) {
  size_t total = 0;
  auto add = [&](size_t b) { total += (b + 255u) & ~(size_t)255u; };
  const size_t row_bytes = (size_t)dim * elem_bytes(store);
  const int cpl = pick_cpl((uint32_t)((row_bytes + 15) / 16));
  const size_t stride = (size_t)8 * (size_t)cpl * 16;
  if (!rows_ready && !(dtype == store && stride == row_bytes && (reinterpret_cast<uintptr_t>(d_data) & 15u) == 0))
    add(stride * N);  // padded or converted rows
  const size_t items = std::max<size_t>((size_t)N * R, 1);
  uint32_t parts = 1, per = 0;
  reverse_parts(N, R, &parts, &per);
  const size_t sort_items = std::max<size_t>(parts == 1 ? items : (size_t)per * R, std::max(N, 1u));
  add((size_t)N * 4);               // deg_work
  add((size_t)N * C * 4);           // work
  add((size_t)N * C * 4);           // wd
  for (int i = 0; i < 4; ++i) add(sort_items * 4);  // keys[2], vals[2]
  add(items * 4);                   // snap
  add(((size_t)N + 1) * 4);         // offs
  if (parts > 1) {                  // split sort
    add(items * 4);                 // pvals
    add((size_t)parts * ((size_t)N + 1) * 4);
    add(((size_t)N + 1) * 8);       // offs64
    add(items * 4);                 // src_sorted
    add(items * 4);                 // snap_sorted
  }
  add(sizeof(VCounters) * kCtrStripes);
  add(sizeof(VCounters));           // summed counters (the prune bound's choice for iteration 1)
  add(kMedoidCandidates * 4);       // scores
  add(kMedoidCandidates * 4);       // cands
  add((size_t)N * kQChunks * 16);   // code rows of the bound
  add((size_t)std::min(locality_cells(store), N) * 4);  // pivots
  add((size_t)N * 4);               // order
  for (size_t n : {(size_t)N, sort_items}) {  // the schedule's sort, then the reverse sort
    const size_t tiles = (n + kRadixTile - 1) / kRadixTile;
    add(tiles * 256 * 4);           // histograms
    size_t levels = 0, m = tiles * 256;
    while (true) {
      const size_t t = (m + kScanTile - 1) / kScanTile;
      levels += t;
      if (t <= 1) break;
      m = t;
    }
    add(std::max<size_t>(levels * 4, 256));  // scan partials
  }
  return total;
}

// Build on device rows into the caller's device graph (N x R) and degrees
// (N). With noalloc, every device buffer comes from this GPU's scratch array,
// the work runs on the null stream and no timing event is created (the stage
// times of the kernel profile read 0; its counters are kept). Callers hold g_mu.
static int resident_build(const void* d_data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t L,
                          uint32_t C, uint32_t STEPS, uint32_t* d_graph, uint32_t* d_degree, bool noalloc) {
  if (d_data == nullptr || d_graph == nullptr || d_degree == nullptr) {
    std::fprintf(stderr, "[gpu_vamana_build] null input pointer.\n");
    return -1;
  }
  if (dtype != DANCE_F32 && dtype != DANCE_U8 && dtype != DANCE_F16) {
    std::fprintf(stderr, "[gpu_vamana_build] unsupported dtype %d\n", dtype);
    return -1;
  }
  DCHECK(validate(N, dim, R, L, C, STEPS));
  const double t0 = now_sec();
  const Profile prof = kProfiles[profile_index_locked()];
  const int store = (dtype == DANCE_F32 && prof.fp16) ? DANCE_F16 : dtype;
  DCHECK(check_width(dim, store));
  Arena arena;
  if (noalloc) {
    const size_t need = resident_build_bytes(d_data, dtype, store, N, dim, R, C);
    if (need > kScratchBytes) {
      std::fprintf(stderr,
                   "[gpu_vamana_build] allocation-free build: N=%u dim=%u R=%u C=%u needs %zu bytes of scratch, "
                   "above its maximum of %zu bytes\n",
                   N, dim, R, C, need, kScratchBytes);
      return -1;
    }
    void* base = nullptr;
    DCHECK(scratch_base(&base));
    arena = Arena{static_cast<char*>(base), kScratchBytes, 0};
  }
  ArenaScope scope(noalloc ? &arena : tl_arena);
  hipStream_t s = nullptr;  // the null stream unless a stream of our own is made
  if (!noalloc) DHIP(hipStreamCreate(&s));
  struct StreamGuard {
    hipStream_t s;
    ~StreamGuard() {
      if (s) (void)hipStreamDestroy(s);
    }
  } sg{s};
  Rows rows;
  DCHECK(setup_rows(rows, d_data, true, dtype, store, N, dim, s));
  State st;
  // The caller's graph and degree buffers are the build's current graph.
  st.cur.p = d_graph;
  st.deg_cur.p = d_degree;
  GPUVamanaStats stats{};
  DanceKernelProfile kp{};
  uint32_t medoid = 0;
  int r = run_build(rows, R, L, C, STEPS, prof, st, s, &stats, &kp, &medoid, !noalloc);
  st.cur.release();
  st.deg_cur.release();
  if (r != 0) return r;
  DHIP(hipStreamSynchronize(s));
  stats.gpu_build_seconds = now_sec() - t0;
  g_last_stats = stats;
  g_last_medoid = medoid;
  g_last_prof = kp;
  return 0;
}

// ---------------------------------------------------------------------------
// Stitched build: per-label standard builds stitched into one global graph
// (reference apps/utils/gpu_stitched_vamana_index.cpp:276-341).
// ---------------------------------------------------------------------------
static DanceStitchedStats g_last_stitched{};

// Device memory in use on the current GPU (total - free), 0 if unknown.
static uint64_t device_used_bytes() {
  size_t fr = 0, tot = 0;
  return hipMemGetInfo(&fr, &tot) == hipSuccess && tot >= fr ? (uint64_t)(tot - fr) : 0u;
}

struct StitchedIn {
  const void* data;  // N x dim rows of dtype (device or host)
  bool data_on_device;
  int dtype;
  uint32_t N, dim;
  const uint32_t* label_offsets;  // host, num_labels + 1
  const uint32_t* label_points;   // host, ascending point ids per label
  uint32_t num_labels;
  uint32_t Rs, Ls, C, steps, Rout, row_cap;
  uint32_t* graph;  // N x row_cap (device or host)
  uint32_t* degree;
  bool out_on_device;
  uint32_t* medoids;  // host, num_labels
};

// Local rows of a label in the build's padded layout: row i is point ids[i]
// of the packed input, converted to the stored type.
static int gather_label_rows(const void* src, int dtype, int store, uint32_t dim, const uint32_t* d_ids, uint32_t m,
                             uint32_t stride_elems, void* dst, hipStream_t s) {
  const uint64_t total = (uint64_t)m * stride_elems;
  if (total == 0) return 0;
  const dim3 grid = grid_dims((total + 255) / 256, 256), block(256);
  if (dtype == DANCE_F32 && store == DANCE_F32)
    hipLaunchKernelGGL((k_gather_rows<float, float>), grid, block, 0, s, static_cast<const float*>(src), dim, d_ids, m,
                       static_cast<float*>(dst), stride_elems);
  else if (dtype == DANCE_F32 && store == DANCE_F16)
    hipLaunchKernelGGL((k_gather_rows<float, _Float16>), grid, block, 0, s, static_cast<const float*>(src), dim, d_ids,
                       m, static_cast<_Float16*>(dst), stride_elems);
  else if (dtype == DANCE_F16)
    hipLaunchKernelGGL((k_gather_rows<_Float16, _Float16>), grid, block, 0, s, static_cast<const _Float16*>(src), dim,
                       d_ids, m, static_cast<_Float16*>(dst), stride_elems);
  else
    hipLaunchKernelGGL((k_gather_rows<uint8_t, uint8_t>), grid, block, 0, s, static_cast<const uint8_t*>(src), dim,
                       d_ids, m, static_cast<uint8_t*>(dst), stride_elems);
  DHIP(hipGetLastError());
  return 0;
}

// Worker threads (streams) of the stitched build: DANCE_STITCHED_WORKERS,
// default 8, 1..16 (c5 stitched, 100 labels of ~10k rows: 481 ms with 1,
// 302 ms with 4, 289 ms with 8). Results do not depend on it.
static uint32_t stitched_workers() {
  const char* e = std::getenv("DANCE_STITCHED_WORKERS");
  const uint32_t v = e && e[0] ? (uint32_t)std::strtoul(e, nullptr, 10) : 8u;
  return std::min(std::max(v, 1u), 16u);
}

// Callers hold g_mu (the workers take no lock: they touch only their own
// arena, stream and staging slices).
static int stitched_build(const StitchedIn& in) {
  const double t0 = now_sec();
  g_last_stitched = DanceStitchedStats{};
  if (!in.data || !in.label_offsets || (in.num_labels && !in.label_points) || !in.graph || !in.degree ||
      (in.num_labels && !in.medoids)) {
    std::fprintf(stderr, "[gpu_stitched] null input pointer.\n");
    return -1;
  }
  if (in.dtype != DANCE_F32 && in.dtype != DANCE_U8 && in.dtype != DANCE_F16) {
    std::fprintf(stderr, "[gpu_stitched] unsupported dtype %d\n", in.dtype);
    return -1;
  }
  if (in.N == 0 || in.dim == 0) {
    std::fprintf(stderr, "[gpu_stitched] invalid parameters N=%u dim=%u\n", in.N, in.dim);
    return -1;
  }
  // Label postings: monotone offsets, point ids in range; labels per point
  // bound the global row length.
  const uint32_t* off = in.label_offsets;
  if (off[0] != 0) {
    std::fprintf(stderr, "[gpu_stitched] label_offsets[0] must be 0\n");
    return -1;
  }
  uint32_t m_max = 0, m_min = UINT32_MAX;
  std::vector<uint32_t> per_point(in.N, 0);
  for (uint32_t l = 0; l < in.num_labels; ++l) {
    if (off[l + 1] < off[l]) {
      std::fprintf(stderr, "[gpu_stitched] label_offsets must not decrease\n");
      return -1;
    }
    const uint32_t m = off[l + 1] - off[l];
    for (uint32_t k = off[l]; k < off[l + 1]; ++k) {
      const uint32_t p = in.label_points[k];
      if (p >= in.N || (k > off[l] && p <= in.label_points[k - 1])) {
        std::fprintf(stderr, "[gpu_stitched] label %u: point ids must be ascending and below N\n", l);
        return -1;
      }
      ++per_point[p];
    }
    if (m) {
      m_max = std::max(m_max, m);
      m_min = std::min(m_min, m);
    }
  }
  const uint32_t take = std::min(in.Rs, in.Rout);
  const uint32_t most = in.N ? *std::max_element(per_point.begin(), per_point.end()) : 0;
  if ((uint64_t)most * take > in.row_cap || in.row_cap > 256 || in.row_cap == 0) {
    std::fprintf(stderr,
                 "[gpu_stitched] row_cap=%u: rows need %llu slots (%u labels x %u) and at most 256 are supported\n",
                 in.row_cap, (unsigned long long)most * take, most, take);
    return -1;
  }
  uint32_t steps = in.steps;
  if (m_max) DCHECK(validate(m_max, in.dim, in.Rs, in.Ls, in.C, steps));
  const Profile prof = kProfiles[profile_index_locked()];
  const int store = (in.dtype == DANCE_F32 && prof.fp16) ? DANCE_F16 : in.dtype;
  DCHECK(check_width(in.dim, store));

  hipStream_t s = nullptr;
  DHIP(hipStreamCreate(&s));
  struct StreamGuard {
    hipStream_t s;
    ~StreamGuard() {
      if (s) (void)hipStreamDestroy(s);
    }
  } sg{s};
  const size_t in_row = (size_t)in.dim * elem_bytes(in.dtype);
  DevBuf up_data, d_pts, d_graph, d_deg, d_ctr;
  const void* src = in.data;
  if (!in.data_on_device) {
    DCHECK(up_data.alloc(in_row * in.N));
    DHIP(hipMemcpyAsync(up_data.p, in.data, in_row * in.N, hipMemcpyHostToDevice, s));
    src = up_data.p;
  }
  const uint32_t total = in.num_labels ? off[in.num_labels] : 0;
  DCHECK(d_pts.alloc(std::max<size_t>(total, 1) * 4));
  if (total) DHIP(hipMemcpyAsync(d_pts.p, in.label_points, (size_t)total * 4, hipMemcpyHostToDevice, s));
  uint32_t* gg = in.graph;
  uint32_t* gd = in.degree;
  const size_t gcells = (size_t)in.N * in.row_cap;
  if (!in.out_on_device) {
    DCHECK(d_graph.alloc(gcells * 4));
    DCHECK(d_deg.alloc((size_t)in.N * 4));
    gg = d_graph.as<uint32_t>();
    gd = d_deg.as<uint32_t>();
  }
  hipLaunchKernelGGL(k_fill_u32, grid_dims(((uint64_t)gcells + 255) / 256, 256), dim3(256), 0, s, gg, (uint64_t)gcells,
                     DANCE_INV);
  hipLaunchKernelGGL(k_fill_u32, dim3((in.N + 255) / 256), dim3(256), 0, s, gd, (uint64_t)in.N, 0u);
  DCHECK(d_ctr.alloc(3 * 8));
  hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(64), 0, s, d_ctr.as<uint32_t>(), (uint64_t)6, 0u);
  DHIP(hipGetLastError());

  // The per-label builds run side by side on W worker threads (stitched_
  // workers()), each with its own stream and its own device arena sized for
  // the largest label (rows and all of the build's buffers). Small labels
  // leave most of the GPU idle, so several in flight keep it busy. Each
  // label's local graph lands in a staging buffer (label l at off[l] rows);
  // the remaps into the global rows then run on this stream in label order,
  // since the cross-label dedupe of multi-label rows depends on that order.
  const size_t row_bytes = (size_t)in.dim * elem_bytes(store);
  const int cpl = pick_cpl((uint32_t)((row_bytes + 15) / 16));
  const uint32_t nch = 8u * (uint32_t)cpl;
  const size_t stride = (size_t)nch * 16;
  auto aligned = [](size_t b) { return (b + 255u) & ~(size_t)255u; };
  const size_t arena_bytes = m_max ? aligned(stride * m_max) +
                                         resident_build_bytes(nullptr, store, store, m_max, in.dim, in.Rs, in.C, true)
                                   : 0;
  uint32_t nonempty = 0;
  for (uint32_t l = 0; l < in.num_labels; ++l) nonempty += off[l + 1] > off[l] ? 1u : 0u;
  const uint32_t W = std::max(1u, std::min(stitched_workers(), nonempty));
  std::vector<DevBuf> arenas(W);
  for (auto& a : arenas) DCHECK(a.alloc(arena_bytes));
  DevBuf stage_g, stage_d;
  DCHECK(stage_g.alloc(std::max<size_t>(total, 1) * in.Rs * 4));
  DCHECK(stage_d.alloc(std::max<size_t>(total, 1) * 4));
  DHIP(hipStreamSynchronize(s));  // uploads and fills done before the workers read them
  DanceStitchedStats st{};
  st.labels = in.num_labels;
  st.label_npts_min = m_max ? m_min : 0;
  st.label_npts_max = m_max;
  st.memberships = total;
  st.row_cap = in.row_cap;
  const double t_setup = now_sec();
  int device = 0;
  DHIP(hipGetDevice(&device));
  std::atomic<uint64_t> peak_used{device_used_bytes()};  // arenas and staging are allocated by now
  std::vector<uint32_t> local_medoid(in.num_labels, 0);
  std::atomic<uint32_t> next{0};
  std::atomic<int> failed{0};
  struct WorkerTimes {
    double materialize = 0, build_sum = 0, build_max = 0;
  };
  std::vector<WorkerTimes> times(W);
  // One label on worker w's stream: gather its rows, build, leave the local
  // graph in the staging buffer.
  auto build_label = [&](uint32_t w, uint32_t l, hipStream_t ws) -> int {
    const uint32_t m = off[l + 1] - off[l];
    Arena arena{arenas[w].as<char>(), arena_bytes, 0};
    ArenaScope scope(&arena);
    const uint32_t* ids = d_pts.as<uint32_t>() + off[l];
    const double tg = now_sec();
    Rows rows;
    DCHECK(rows.owned.alloc(stride * m));
    DCHECK(gather_label_rows(src, in.dtype, store, in.dim, ids, m, (uint32_t)(stride / elem_bytes(store)),
                             rows.owned.p, ws));
    rows.dtype = store;
    rows.N = m;
    rows.dim = in.dim;
    rows.rs.rows = rows.owned.as<const uint4>();
    rows.rs.stride16 = nch;
    rows.rs.nch = nch;
    rows.rs.tail16 = (store == DANCE_F16 && (in.dim & 1u)) ? (int32_t)((in.dim - 1u) / 2u) : -1;
    DHIP(hipStreamSynchronize(ws));
    const double tb = now_sec();
    times[w].materialize += tb - tg;
    State lst;  // the local graph and degrees are slices of the staging buffers
    lst.cur.p = stage_g.as<uint32_t>() + (size_t)off[l] * in.Rs;
    lst.cur.bytes = (size_t)m * in.Rs * 4;
    lst.cur.borrowed = true;
    lst.deg_cur.p = stage_d.as<uint32_t>() + off[l];
    lst.deg_cur.bytes = (size_t)m * 4;
    lst.deg_cur.borrowed = true;
    DCHECK(run_build(rows, in.Rs, in.Ls, in.C, steps, prof, lst, ws, nullptr, nullptr, &local_medoid[l], false));
    const double dt = now_sec() - tb;
    const uint64_t used = device_used_bytes();
    for (uint64_t cur = peak_used.load(); used > cur && !peak_used.compare_exchange_weak(cur, used);) {
    }
    times[w].build_sum += dt;
    times[w].build_max = std::max(times[w].build_max, dt);
    return 0;
  };
  auto worker = [&](uint32_t w) {
    if (hipSetDevice(device) != hipSuccess) {
      failed = 1;
      return;
    }
    hipStream_t ws = nullptr;
    if (hipStreamCreate(&ws) != hipSuccess) {
      failed = 1;
      return;
    }
    for (uint32_t l; !failed && (l = next.fetch_add(1)) < in.num_labels;)
      if (off[l + 1] > off[l] && build_label(w, l, ws) != 0) failed = 1;
    (void)hipStreamDestroy(ws);
  };
  {
    std::vector<std::thread> pool;
    for (uint32_t w = 1; w < W; ++w) pool.emplace_back(worker, w);
    worker(0);
    for (auto& t : pool) t.join();
  }
  if (failed) return -1;
  for (const auto& t : times) {
    st.materialize_seconds += t.materialize;
    st.build_sum_seconds += t.build_sum;
    st.build_max_seconds = std::max(st.build_max_seconds, t.build_max);
  }
  const double tr = now_sec();
  for (uint32_t l = 0; l < in.num_labels; ++l) {
    const uint32_t m = off[l + 1] - off[l];
    if (m == 0) {
      in.medoids[l] = DANCE_INV;
      continue;
    }
    RemapArgs ra{stage_g.as<uint32_t>() + (size_t)off[l] * in.Rs, stage_d.as<uint32_t>() + off[l],
                 d_pts.as<uint32_t>() + off[l], m, in.Rs, in.Rout, gg, gd, in.row_cap,
                 d_ctr.as<unsigned long long>()};
    hipLaunchKernelGGL(k_stitch_remap, grid_dims(((uint64_t)m + kRemapWaves - 1) / kRemapWaves, 64 * kRemapWaves),
                       dim3(64 * kRemapWaves), 0, s, ra);
    DHIP(hipGetLastError());
    in.medoids[l] = in.label_points[off[l] + (local_medoid[l] < m ? local_medoid[l] : 0u)];
  }
  DHIP(hipStreamSynchronize(s));
  st.remap_seconds = now_sec() - tr;
  st.peak_gpu_mem_gb = (double)std::max<uint64_t>(peak_used.load(), device_used_bytes()) / (1024.0 * 1024.0 * 1024.0);
  unsigned long long c3[3] = {0, 0, 0};
  DHIP(hipMemcpyAsync(c3, d_ctr.p, sizeof(c3), hipMemcpyDeviceToHost, s));
  DHIP(hipStreamSynchronize(s));
  if (!in.out_on_device) {
    DCHECK(copy_pageable(in.graph, gg, gcells * 4, hipMemcpyDeviceToHost));
    DCHECK(copy_pageable(in.degree, gd, (size_t)in.N * 4, hipMemcpyDeviceToHost));
  }
  st.remap_invalid_local_ids = c3[0];
  st.remap_self_loops = c3[1];
  st.remap_duplicate_edges = c3[2];
  st.setup_seconds = t_setup - t0;
  st.total_seconds = now_sec() - t0;
  g_last_stitched = st;
  return 0;
}

extern "C" {

int gpu_vamana_vnew2_build(const uint8_t* h_data, uint32_t N, uint32_t dim, uint32_t R, uint32_t L, uint32_t C,
                           uint32_t STEPS, uint32_t* h_graph, uint32_t* h_degree) {
  return build_host<uint8_t>(h_data, DANCE_U8, N, dim, R, L, C, STEPS, h_graph, h_degree, nullptr, nullptr, nullptr);
}

int gpu_vamana_vnew2_build_float(const float* h_data, uint32_t N, uint32_t dim, uint32_t R, uint32_t L, uint32_t C,
                                 uint32_t STEPS, uint32_t* h_graph, uint32_t* h_degree) {
  return build_host<float>(h_data, DANCE_F32, N, dim, R, L, C, STEPS, h_graph, h_degree, nullptr, nullptr, nullptr);
}

// The v8 builder (gpu_vamana_uint8.cu:3093-3120): the reference converts float
// input to binary16 on the host under the fp16 profiles (:3100-3115); the same
// round-to-nearest-even conversion runs here on the device after the upload.
int gpu_vamana_build(const uint8_t* h_data, uint32_t N, uint32_t dim, uint32_t R, uint32_t L, uint32_t C,
                     uint32_t STEPS, uint32_t* h_graph, uint32_t* h_degree) {
  return build_host<uint8_t>(h_data, DANCE_U8, N, dim, R, L, C, STEPS, h_graph, h_degree, nullptr, nullptr, nullptr,
                             Builder::v8);
}

int gpu_vamana_build_float(const float* h_data, uint32_t N, uint32_t dim, uint32_t R, uint32_t L, uint32_t C,
                           uint32_t STEPS, uint32_t* h_graph, uint32_t* h_degree) {
  return build_host<float>(h_data, DANCE_F32, N, dim, R, L, C, STEPS, h_graph, h_degree, nullptr, nullptr, nullptr,
                           Builder::v8);
}

int gpu_vamana_vnew2_build_device(const uint8_t* h_data, uint32_t N, uint32_t dim, uint32_t R, uint32_t L, uint32_t C,
                                  uint32_t STEPS, uint8_t** d_data, uint32_t** d_graph, uint32_t** d_degree) {
  if (d_data == nullptr || d_graph == nullptr || d_degree == nullptr) {
    std::fprintf(stderr, "[gpu_vamana_build] null output pointer.\n");
    return -1;
  }
  void* dd = nullptr;
  int r = build_host<uint8_t>(h_data, DANCE_U8, N, dim, R, L, C, STEPS, nullptr, nullptr, &dd, d_graph, d_degree);
  if (r == 0) *d_data = static_cast<uint8_t*>(dd);
  return r;
}

int gpu_vamana_vnew2_build_device_float(const float* h_data, uint32_t N, uint32_t dim, uint32_t R, uint32_t L,
                                        uint32_t C, uint32_t STEPS, float** d_data, uint32_t** d_graph,
                                        uint32_t** d_degree) {
  if (d_data == nullptr || d_graph == nullptr || d_degree == nullptr) {
    std::fprintf(stderr, "[gpu_vamana_build] null output pointer.\n");
    return -1;
  }
  void* dd = nullptr;
  int r = build_host<float>(h_data, DANCE_F32, N, dim, R, L, C, STEPS, nullptr, nullptr, &dd, d_graph, d_degree);
  if (r == 0) *d_data = static_cast<float*>(dd);
  return r;
}

uint32_t dance_struct_sizes(uint64_t* sizes, uint32_t count) {
  const uint64_t all[7] = {sizeof(GPUVamanaStats),   sizeof(DanceKernelProfile), sizeof(GPUFilteredVamanaStats),
                           sizeof(DanceFilteredProfile), sizeof(DanceSearchStats), sizeof(DanceMergeStats),
                           sizeof(DanceStitchedStats)};
  for (uint32_t i = 0; sizes && i < count && i < 7; ++i) sizes[i] = all[i];
  return 7;
}

int dance_stitched_build(const void* h_data, int dtype, uint32_t num_points, uint32_t dim,
                         const uint32_t* label_offsets, const uint32_t* label_points, uint32_t num_labels,
                         uint32_t R_small, uint32_t L_small, uint32_t C, uint32_t STEPS, uint32_t R_stitched,
                         uint32_t row_cap, uint32_t* h_graph, uint32_t* h_degree, uint32_t* label_medoids) {
  std::lock_guard<std::mutex> lk(g_mu);
  return stitched_build(StitchedIn{h_data, false, dtype, num_points, dim, label_offsets, label_points, num_labels,
                                   R_small, L_small, C, STEPS, R_stitched, row_cap, h_graph, h_degree, false,
                                   label_medoids});
}

int dance_stitched_build_resident(const void* d_data, int dtype, uint32_t num_points, uint32_t dim,
                                  const uint32_t* label_offsets, const uint32_t* label_points, uint32_t num_labels,
                                  uint32_t R_small, uint32_t L_small, uint32_t C, uint32_t STEPS,
                                  uint32_t R_stitched, uint32_t row_cap, uint32_t* d_graph, uint32_t* d_degree,
                                  uint32_t* label_medoids) {
  std::lock_guard<std::mutex> lk(g_mu);
  return stitched_build(StitchedIn{d_data, true, dtype, num_points, dim, label_offsets, label_points, num_labels,
                                   R_small, L_small, C, STEPS, R_stitched, row_cap, d_graph, d_degree, true,
                                   label_medoids});
}

void dance_get_last_stitched_stats(DanceStitchedStats* stats) {
  if (stats) *stats = g_last_stitched;
}

uint32_t gpu_vamana_vnew2_get_last_medoid(void) { return g_last_medoid; }
void gpu_vamana_vnew2_get_last_stats(GPUVamanaStats* stats) {
  if (stats) *stats = g_last_stats;
}
uint32_t gpu_vamana_get_last_medoid(void) { return g_last_medoid_v8; }
void gpu_vamana_get_last_stats(GPUVamanaStats* stats) {
  if (stats) *stats = g_last_stats_v8;
}

// ===========================================================================
// Extensions (include/dance_hip.h)
// ===========================================================================
int dance_vamana_build_resident(const void* d_data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t L,
                                uint32_t C, uint32_t STEPS, uint32_t* d_graph, uint32_t* d_degree) {
  std::lock_guard<std::mutex> lk(g_mu);
  return resident_build(d_data, dtype, N, dim, R, L, C, STEPS, d_graph, d_degree, false);
}

int dance_vamana_build_resident_noalloc(const void* d_data, int dtype, uint32_t N, uint32_t dim, uint32_t R,
                                        uint32_t L, uint32_t C, uint32_t STEPS, uint32_t* d_graph,
                                        uint32_t* d_degree) {
  std::lock_guard<std::mutex> lk(g_mu);
  return resident_build(d_data, dtype, N, dim, R, L, C, STEPS, d_graph, d_degree, true);
}

void dance_get_last_kernel_profile(DanceKernelProfile* p) {
  if (p) *p = g_last_prof;
}

int dance_set_profile(const char* name) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (name == nullptr) return -1;
  for (int i = 0; i < 4; ++i)
    if (std::strcmp(name, kProfiles[i].name) == 0) {
      g_profile = i;
      return 0;
    }
  std::fprintf(stderr, "[dance_hip] unknown profile '%s'\n", name);
  return -1;
}

const char* dance_get_profile(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  return kProfiles[profile_index_locked()].name;
}

int dance_stage_distances(const void* h_data, int dtype, uint32_t N, uint32_t dim, const uint32_t* a,
                          const uint32_t* b, uint64_t n, float* out) {
  if (!h_data || !a || !b || !out || N == 0 || dim == 0) return -1;
  for (uint64_t i = 0; i < n; ++i)
    if (a[i] >= N || b[i] >= N) {
      std::fprintf(stderr, "[dance_hip] distance index out of range\n");
      return -1;
    }
  StageCtx cx;
  DCHECK(cx.open(h_data, dtype, N, dim));
  DevBuf da, db, dout;
  DCHECK(da.alloc(std::max<uint64_t>(n, 1) * 4));
  DCHECK(db.alloc(std::max<uint64_t>(n, 1) * 4));
  DCHECK(dout.alloc(std::max<uint64_t>(n, 1) * 4));
  DCHECK(up(da.p, a, n * 4, cx.s));
  DCHECK(up(db.p, b, n * 4, cx.s));
  const int cpl = pick_cpl(cx.rows.rs.nch);
  const uint64_t waves = (n + 63) / 64;
  DCHECK(with_dt_cpl(dtype, cpl, [&](auto dt, auto c) {
    if (waves == 0) return 0;
    hipLaunchKernelGGL((k_pair_dist<decltype(dt)::value, decltype(c)::value>),
                       dim3((uint32_t)((waves + kWavesPerBlock - 1) / kWavesPerBlock)), dim3(kBlock), 0, cx.s,
                       cx.rows.rs, da.as<uint32_t>(), db.as<uint32_t>(), n, dout.as<float>());
    DHIP(hipGetLastError());
    return 0;
  }));
  DCHECK(down(out, dout.p, n * 4, cx.s));
  DHIP(hipStreamSynchronize(cx.s));
  return 0;
}

int dance_stage_qbound(const void* h_data, int dtype, uint32_t N, uint32_t dim, const uint32_t* a, const uint32_t* b,
                       const float* T, uint64_t n, uint32_t* flags) {
  if (!h_data || !a || !b || !T || !flags || N == 0 || dim == 0) return -1;
  for (uint64_t i = 0; i < n; ++i)
    if (a[i] >= N || b[i] >= N) {
      std::fprintf(stderr, "[dance_hip] bound index out of range\n");
      return -1;
    }
  StageCtx cx;
  DCHECK(cx.open(h_data, dtype, N, dim));
  DevBuf qbuf, da, db, dt, dout;
  QBoundSet qb{};
  DCHECK(build_qbound(cx.rows, qbuf, cx.s, &qb));
  if (!qb.rows) {
    std::fprintf(stderr, "[dance_hip] no distance bound for this row type / width (or DANCE_QBOUND=0)\n");
    return -1;
  }
  const uint64_t m = std::max<uint64_t>(n, 1);
  DCHECK(da.alloc(m * 4));
  DCHECK(db.alloc(m * 4));
  DCHECK(dt.alloc(m * 4));
  DCHECK(dout.alloc(m * 4));
  DCHECK(up(da.p, a, n * 4, cx.s));
  DCHECK(up(db.p, b, n * 4, cx.s));
  DCHECK(up(dt.p, T, n * 4, cx.s));
  const uint64_t waves = (n + 63) / 64;
  if (waves) {
    hipLaunchKernelGGL(k_qbound_pairs, dim3((uint32_t)((waves + kWavesPerBlock - 1) / kWavesPerBlock)), dim3(kBlock),
                       0, cx.s, qb, da.as<uint32_t>(), db.as<uint32_t>(), dt.as<float>(), n, dout.as<uint32_t>());
    DHIP(hipGetLastError());
  }
  DCHECK(down(flags, dout.p, n * 4, cx.s));
  DHIP(hipStreamSynchronize(cx.s));
  return 0;
}

int dance_stage_insert_bound(const void* h_data, int dtype, uint32_t N, uint32_t dim, const uint32_t* a,
                             const uint32_t* b, const float* T0, float alpha, uint64_t n, uint32_t* out) {
  if (!h_data || !a || !b || !T0 || !out || N == 0 || dim == 0) return -1;
  for (uint64_t i = 0; i < n; ++i)
    if (a[i] >= N || b[i] >= N) {
      std::fprintf(stderr, "[dance_hip] bound index out of range\n");
      return -1;
    }
  StageCtx cx;
  DCHECK(cx.open(h_data, dtype, N, dim));
  DevBuf qbuf, da, db, dt, dout;
  QBoundSet qb{};
  DCHECK(build_qbound(cx.rows, qbuf, cx.s, &qb));
  if (!qb.rows) {
    std::fprintf(stderr, "[dance_hip] no distance bound for this row type / width (or DANCE_QBOUND=0)\n");
    return -1;
  }
  const uint64_t m = std::max<uint64_t>(n, 1);
  DCHECK(da.alloc(m * 4));
  DCHECK(db.alloc(m * 4));
  DCHECK(dt.alloc(m * 4));
  DCHECK(dout.alloc(m * 4));
  DCHECK(up(da.p, a, n * 4, cx.s));
  DCHECK(up(db.p, b, n * 4, cx.s));
  DCHECK(up(dt.p, T0, n * 4, cx.s));
  const uint64_t waves = (n + 63) / 64;
  if (waves) {
    const dim3 grid((uint32_t)((waves + kWavesPerBlock - 1) / kWavesPerBlock));
    if (cx.rows.dtype == DANCE_F16)
      hipLaunchKernelGGL(k_insert_bound_pairs<DANCE_F16>, grid, dim3(kBlock), 0, cx.s, qb, da.as<uint32_t>(),
                         db.as<uint32_t>(), dt.as<float>(), alpha, n, dout.as<uint32_t>());
    else
      hipLaunchKernelGGL(k_insert_bound_pairs<DANCE_F32>, grid, dim3(kBlock), 0, cx.s, qb, da.as<uint32_t>(),
                         db.as<uint32_t>(), dt.as<float>(), alpha, n, dout.as<uint32_t>());
    DHIP(hipGetLastError());
  }
  DCHECK(down(out, dout.p, n * 4, cx.s));
  DHIP(hipStreamSynchronize(cx.s));
  return 0;
}

int dance_stage_medoid(const void* h_data, int dtype, uint32_t N, uint32_t dim, float* scores, uint32_t* cands,
                       uint32_t* medoid) {
  if (!h_data || N == 0 || dim == 0) return -1;
  StageCtx cx;
  DCHECK(cx.open(h_data, dtype, N, dim));
  const uint32_t nc = std::min(kMedoidCandidates, N), ns = std::min(kMedoidSamples, N);
  DevBuf sc, ca;
  DCHECK(sc.alloc(nc * 4));
  DCHECK(ca.alloc(nc * 4));
  DCHECK(launch_medoid(cx.rows, cx.s, sc.as<float>(), ca.as<uint32_t>(), nc, ns));
  std::vector<float> hs(nc);
  std::vector<uint32_t> hc(nc);
  DCHECK(down(hs.data(), sc.p, nc * 4, cx.s));
  DCHECK(down(hc.data(), ca.p, nc * 4, cx.s));
  DHIP(hipStreamSynchronize(cx.s));
  uint32_t best = DANCE_INV;
  float bs = FLT_MAX;
  for (uint32_t i = 0; i < nc; ++i)
    if (hs[i] < bs) {
      bs = hs[i];
      best = i;
    }
  if (scores) std::memcpy(scores, hs.data(), nc * 4);
  if (cands) std::memcpy(cands, hc.data(), nc * 4);
  if (medoid) *medoid = best == DANCE_INV ? 0u : hc[best];
  return 0;
}

int dance_stage_init(const void* h_data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t C, uint32_t* cur,
                     uint32_t* deg_cur, uint32_t* work, uint32_t* deg_work, float* wd) {
  if (!h_data || !cur || !deg_cur || !work || !deg_work || !wd || N == 0 || R == 0 || C < R) return -1;
  StageCtx cx;
  DCHECK(cx.open(h_data, dtype, N, dim));
  DCHECK(cx.st.alloc(N, R, C));
  DCHECK(launch_init(cx.rows, cx.st.g(), cx.s));
  return download_state(cx.st, cur, deg_cur, work, deg_work, wd, cx.s);
}

int dance_stage_search(const void* h_data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t L, uint32_t C,
                       uint32_t steps, float alpha, uint32_t start, uint32_t* cur, uint32_t* deg_cur, uint32_t* work,
                       uint32_t* deg_work, float* wd) {
  if (!h_data || !cur || !deg_cur || !work || !deg_work || !wd || N == 0 || R == 0 || C < R || L == 0 || L > 256)
    return -1;
  StageCtx cx;
  DCHECK(cx.open(h_data, dtype, N, dim));
  DCHECK(upload_state(cx.st, N, R, C, cur, deg_cur, work, deg_work, wd, cx.s));
  DevBuf qbuf;
  QBoundSet qb{};
  DCHECK(build_qbound(cx.rows, qbuf, cx.s, &qb));
  DCHECK(launch_search(cx.rows, cx.st.g(), L, steps, alpha, start, nullptr, nullptr, qb, cx.s,
                       (insert_bound_iters() & 1u) != 0, false));  // cur comes from the caller
  return download_state(cx.st, cur, deg_cur, work, deg_work, wd, cx.s);
}

int dance_stage_reverse_merge(const void* h_data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t C,
                              uint32_t* work, uint32_t* deg_work, float* wd, uint32_t heavy_threshold,
                              uint32_t heavy_sample, uint32_t* offsets, uint32_t* ids) {
  if (!h_data || !work || !deg_work || !wd || N == 0 || R == 0 || C < R) return -1;
  StageCtx cx;
  DCHECK(cx.open(h_data, dtype, N, dim));
  DCHECK(upload_state(cx.st, N, R, C, nullptr, nullptr, work, deg_work, wd, cx.s));
  ReverseWs rws;
  DCHECK(rws.alloc(N, R));
  GraphBufs g = cx.st.g();
  RevCsr rev{};
  DCHECK(build_reverse_csr(g, rws, cx.s, &rev));
  std::vector<uint32_t> off((size_t)N + 1);
  if (rev.offs64) {  // split sort: 64-bit offsets, srcs already sources
    std::vector<uint64_t> off64((size_t)N + 1);
    DCHECK(down(off64.data(), rev.offs64, ((size_t)N + 1) * 8, cx.s));
    DHIP(hipStreamSynchronize(cx.s));
    for (size_t t = 0; t <= N; ++t) off[t] = (uint32_t)off64[t];
  } else {
    DCHECK(down(off.data(), rev.offs, ((size_t)N + 1) * 4, cx.s));
    DHIP(hipStreamSynchronize(cx.s));
  }
  if (offsets) std::memcpy(offsets, off.data(), off.size() * 4);
  if (ids) {
    DCHECK(down(ids, rev.srcs, (size_t)off[N] * 4, cx.s));
    DHIP(hipStreamSynchronize(cx.s));
    if (!rev.offs64)
      for (uint32_t e = 0; e < off[N]; ++e) ids[e] /= R;  // forward slot -> source
  }
  Profile prof{"stage", false, heavy_threshold, heavy_sample};
  DCHECK(launch_merge(cx.rows, g, rev, prof, nullptr, nullptr, cx.s));
  return download_state(cx.st, nullptr, nullptr, work, deg_work, wd, cx.s);
}

int dance_stage_prune(const void* h_data, int dtype, uint32_t N, uint32_t dim, uint32_t R, uint32_t C,
                      uint32_t min_degree, float alpha, uint32_t* work, uint32_t* deg_work, float* wd, uint32_t* cur,
                      uint32_t* deg_cur) {
  if (!h_data || !work || !deg_work || !wd || !cur || !deg_cur || N == 0 || R == 0 || C < R) return -1;
  StageCtx cx;
  DCHECK(cx.open(h_data, dtype, N, dim));
  DCHECK(upload_state(cx.st, N, R, C, nullptr, nullptr, work, deg_work, wd, cx.s));
  DevBuf qbuf;
  QBoundSet qb{};
  DCHECK(build_qbound(cx.rows, qbuf, cx.s, &qb));
  // the stage hook runs the kernel the last iteration would use
  DCHECK(launch_prune(cx.rows, cx.st.g(), min_degree, alpha, nullptr, nullptr, qb,
                      ((prune_rank_iters(cx.rows.dtype) >> (kDefaultIters - 1)) & 1u) != 0u, cx.s));
  return download_state(cx.st, cur, deg_cur, work, deg_work, wd, cx.s);
}

int dance_stage_sort_pairs(const uint32_t* keys, const uint32_t* vals, uint64_t n, uint32_t key_bits,
                           uint32_t* out_keys, uint32_t* out_vals) {
  if (!keys || !vals || !out_keys || !out_vals || key_bits > 32) return -1;
  hipStream_t s = nullptr;
  DHIP(hipStreamCreate(&s));
  struct G {
    hipStream_t s;
    ~G() { (void)hipStreamDestroy(s); }
  } gd{s};
  DevBuf k[2], v[2];
  for (int i = 0; i < 2; ++i) {
    DCHECK(k[i].alloc(std::max<uint64_t>(n, 1) * 4));
    DCHECK(v[i].alloc(std::max<uint64_t>(n, 1) * 4));
  }
  DCHECK(up(k[0].p, keys, n * 4, s));
  DCHECK(up(v[0].p, vals, n * 4, s));
  uint32_t* kb[2] = {k[0].as<uint32_t>(), k[1].as<uint32_t>()};
  uint32_t* vb[2] = {v[0].as<uint32_t>(), v[1].as<uint32_t>()};
  SortWorkspace ws;
  int which = 0;
  DCHECK(radix_sort_pairs(kb, vb, n, key_bits, ws, s, &which));
  DCHECK(down(out_keys, kb[which], n * 4, s));
  DCHECK(down(out_vals, vb[which], n * 4, s));
  DHIP(hipStreamSynchronize(s));
  return 0;
}

int dance_stage_scan(const uint32_t* in, uint64_t n, uint32_t* out) {
  if (!in || !out) return -1;
  hipStream_t s = nullptr;
  DHIP(hipStreamCreate(&s));
  struct G {
    hipStream_t s;
    ~G() { (void)hipStreamDestroy(s); }
  } gd{s};
  DevBuf d;
  DCHECK(d.alloc(std::max<uint64_t>(n, 1) * 4));
  DCHECK(up(d.p, in, n * 4, s));
  ScanWorkspace ws;
  DCHECK(scan_exclusive(d.as<uint32_t>(), n, ws, s));
  DCHECK(down(out, d.p, n * 4, s));
  DHIP(hipStreamSynchronize(s));
  return 0;
}

}  // extern "C"
