// Host orchestration of the label-filtered build and the C ABI of
// include/gpu_vamana_filtered.h (+ the dance_filtered_* extensions of
// include/dance_hip.h).
//
// Schedule (gpu_vamana_filtered_build_impl, /root/reference/src/gpu_vamana_filtered.cu:6511-7067,
// canonical_round0_from_host_backbone_typed, :5663-6483):
//   labels + postings upload -> random backbone -> task rows ->
//   3 x (task search -> row kernel (union search, merge, quota, work
//        distances, forward prune) -> reverse count / scan / fill ->
//        exact CSR prune: k_csr for lists <= 256, k_csr_long above) -> [publish: shortlist + prune to PR, reverse
//        CSR, shortlist + prune of the touched rows] -> diagnostics ->
//        download.
//
// Device layout (row-major):
//   rows      N x stride16 x 16 B    fp16 (float input) or u8 vectors
//   ga, gb    N x R u32              graph (round input) / forward graph
//   da, db    N u32                  degrees
//   tids, td  T x keep               task results (T = total labels)
//   roff      N+1 u32                reverse CSR offsets; rids <= N*R sources
//   boff      N+1 u32                scratch offsets of lists > 256 entries
//   bd, brem, bmask  per long-list entry   distances / removed flags / label masks
//   lrows     <= N u32               rows with long lists (k_csr_long, one workgroup each)
// Each round reads ga and writes gb (forward), then writes ga (repaired).
// The publish step (DISKANN_GPU_FILTERED_PUBLISH_DEGREE = PR below R) writes
// its N x PR graph into gb / db; rows of more than 256 candidates use
// boff / bmask (ids) / bd / brem (states) as scratch.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/dance_hip.h"
#include "../../include/gpu_vamana_filtered.h"
#include "filtered_kernels.h"
#include "host_common.h"

static_assert(sizeof(GPUFilteredVamanaStats) == 456, "GPUFilteredVamanaStats layout");
static_assert(offsetof(GPUFilteredVamanaStats, filtered_search_distance_count) == 120, "layout");
static_assert(offsetof(GPUFilteredVamanaStats, avg_common_label_out_degree) == 352, "layout");
static_assert(offsetof(GPUFilteredVamanaStats, out_degree_avg) == 408, "layout");
static_assert(offsetof(GPUFilteredVamanaStats, prune_output_degree_avg) == 432, "layout");
static_assert(offsetof(GPUFilteredVamanaStats, semantic_complete) == 448, "layout");

namespace dance {
namespace {

using namespace filt;

constexpr uint32_t kRounds = 3;         // configured_rounds (:5707)
constexpr uint32_t kBackboneSeed = 42;  // (:6987)
constexpr uint32_t kBackboneDegree = 16;
constexpr uint32_t kStageLabelSync = 6;  // GPU_FILTERED_STAGE_LABEL_SYNC (:65)

std::mutex g_fmu;
GPUFilteredVamanaStats g_fstats{};
DanceFilteredProfile g_fprof{};

struct FParams {
  uint32_t N, dim, R, L, filtered_L, C, STEPS;
  float alpha;
  uint32_t total, num_labels, universal, global_start, rounds;
};

const char* kTag = "[gpu_vamana_filtered]";

// The reference's build log (navigation-policy banner, one line per round,
// the coverage-repair line, the degree percentiles of the published graph;
// gpu_vamana_filtered.cu:5723-5730, :6294-6297, :6325, :94-160) goes to
// stdout unless DANCE_FILTERED_LOG=0. The per-round counts and the
// percentiles cost extra work (a copy of the round's input graph and two
// small kernels), done only while the log is on.
bool filtered_log() {
  const char* e = std::getenv("DANCE_FILTERED_LOG");
  return !(e && e[0] == '0');
}

// Parameter and label checks of gpu_vamana_filtered_build_impl (:6558-6568),
// plus offsets consistency (the reference reads out of bounds otherwise).
int validate(const FParams& p, const uint32_t* off, const uint32_t* lab, const uint32_t* starts) {
  if (!off || !lab || !starts) {
    std::fprintf(stderr, "%s null input pointer.\n", kTag);
    return -1;
  }
  if (p.N == 0 || p.dim == 0 || p.R == 0 || p.L == 0 || p.C < p.R) {
    std::fprintf(stderr, "%s invalid parameters N=%u dim=%u R=%u L=%u C=%u\n", kTag, p.N, p.dim, p.R, p.L, p.C);
    return -1;
  }
  if (p.rounds > kRounds) {
    std::fprintf(stderr, "%s rounds=%u exceeds %u\n", kTag, p.rounds, kRounds);
    return -1;
  }
  if (off[0] != 0 || off[p.N] != p.total) {
    std::fprintf(stderr, "%s label offsets must start at 0 and end at total_label_count=%u\n", kTag, p.total);
    return -1;
  }
  for (uint32_t i = 0; i < p.N; ++i) {
    if (off[i + 1] < off[i]) {
      std::fprintf(stderr, "%s label offsets decrease at point %u\n", kTag, i);
      return -1;
    }
    // sorted unique labels per point (DiskANN canonicalises them, patch:20269-20286)
    for (uint32_t j = off[i] + 1; j < off[i + 1]; ++j)
      if (lab[j] <= lab[j - 1]) {
        std::fprintf(stderr, "%s labels of point %u are not sorted and unique\n", kTag, i);
        return -1;
      }
  }
  // The reverse CSR needs 2R entries per point of the work capacity (:5839-5846).
  if ((uint64_t)p.N * std::min(p.C, kMaxWorkC) < (uint64_t)2 * p.N * p.R) {
    std::fprintf(stderr, "%s GPU work capacity cannot hold exact reverse CSR\n", kTag);
    return 1;
  }
  return 0;
}

struct FState {
  DevBuf off, lab, lab8, sig, gsig, lpo, lpts, starts, task_rows, rorder, torder;
  DevBuf ga, gb, da, db, tids, td;
  DevBuf roff, cursor, rids, boff, bd, brem, bmask, lrows, lsort, lcount;
  DevBuf ctr, d32, d64;
  DevBuf prev_g, prev_d, rcnt, compat, minpl;  // build log only
  size_t big_cap = 0;
  // the output graph: ga / da, or gb / db after the publish step
  uint32_t out_R = 0;
  void* out_g = nullptr;
  void* out_d = nullptr;
};

// DISKANN_GPU_FILTERED_PUBLISH_DEGREE (gpu_vamana_filtered.cu:6328-6331): a
// positive value caps the published degree at min(R, value).
uint32_t publish_degree(uint32_t R) {
  const char* e = std::getenv("DISKANN_GPU_FILTERED_PUBLISH_DEGREE");
  const int v = e ? std::atoi(e) : 0;
  return v > 0 ? std::min(R, (uint32_t)v) : R;
}

// Makes the long-list scratch hold `need` entries.
int ensure_big(FState& st, size_t need) {
  if (need <= st.big_cap) return 0;
  DCHECK(st.bd.alloc(need * 4));
  DCHECK(st.brem.alloc(need));
  DCHECK(st.bmask.alloc(need * 4));
  st.big_cap = need;
  return 0;
}

struct FEvents {
  std::vector<hipEvent_t> ev;
  ~FEvents() {
    for (hipEvent_t e : ev) (void)hipEventDestroy(e);
  }
  hipEvent_t mark(hipStream_t s) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    ev.push_back(e);
    (void)hipEventRecord(e, s);
    return e;
  }
};

float ms_between(hipEvent_t a, hipEvent_t b) {
  float ms = 0.f;
  if (a && b && hipEventElapsedTime(&ms, a, b) == hipSuccess) return ms;
  return 0.f;
}

// Grid of wave-per-item kernels remapped across XCDs (xcd_block): a multiple
// of 8 workgroups, 2-D beyond 2^32 work-items (grid_dims).
dim3 grid_xcd(uint64_t waves) { return grid_dims((waves + kWaves - 1) / kWaves, kBlock, 8); }
uint32_t grid_thr(uint64_t n) { return (uint32_t)((n + 255) / 256); }

void peak_mem(double& peak) {
  size_t fr = 0, tot = 0;
  if (hipMemGetInfo(&fr, &tot) == hipSuccess) peak = std::max(peak, (double)(tot - fr) / (1024.0 * 1024.0 * 1024.0));
}

struct StreamGuard {
  hipStream_t s = nullptr;
  ~StreamGuard() {
    if (s) (void)hipStreamDestroy(s);
  }
};

// canonical_print_round_diagnostics (gpu_vamana_filtered.cu:94-160) over the
// published graph: the per-row figures come from k_degree_profile, the
// percentiles (entry floor(q * (N - 1)) of the ascending values) from the host.
int print_degree_profile(FState& st, const Labels& Ld, uint32_t N, hipStream_t s) {
  const double t0 = now_sec();
  const uint32_t R = st.out_R;
  DCHECK(st.compat.alloc((size_t)N * 4));
  DCHECK(st.minpl.alloc((size_t)N * 4));
  hipLaunchKernelGGL(k_degree_profile, dim3(grid_thr(N)), dim3(256), 0, s,
                     Graph{N, R, static_cast<const uint32_t*>(st.out_g), static_cast<const uint32_t*>(st.out_d)}, Ld,
                     st.compat.as<uint32_t>(), st.minpl.as<uint32_t>());
  DHIP(hipGetLastError());
  std::vector<uint32_t> deg(N), compat(N), minpl(N);
  DHIP(hipMemcpyAsync(deg.data(), st.out_d, (size_t)N * 4, hipMemcpyDeviceToHost, s));
  DHIP(hipMemcpyAsync(compat.data(), st.compat.p, (size_t)N * 4, hipMemcpyDeviceToHost, s));
  DHIP(hipMemcpyAsync(minpl.data(), st.minpl.p, (size_t)N * 4, hipMemcpyDeviceToHost, s));
  DHIP(hipStreamSynchronize(s));
  uint64_t deg_sum = 0, at_R = 0, compat_sum = 0, minpl_sum = 0;
  for (uint32_t r = 0; r < N; ++r) {
    const uint32_t d = std::min(deg[r], R);
    deg_sum += d;
    at_R += d == R;
    compat_sum += compat[r];
    minpl_sum += minpl[r];
  }
  auto pct = [N](std::vector<uint32_t>& v, double q) {
    const size_t k = (size_t)(q * (double)(N - 1));
    std::nth_element(v.begin(), v.begin() + k, v.end());
    return v[k];
  };
  uint32_t pd[3], pc[3], pm[3];
  const double qs[3] = {0.50, 0.95, 0.99};
  for (int i = 0; i < 3; ++i) {
    pd[i] = pct(deg, qs[i]);
    pc[i] = pct(compat, qs[i]);
    pm[i] = pct(minpl, qs[i]);
  }
  const double n = (double)N;
  std::printf("[gpu_vamana_filtered_canonical_degree] avg=%.3f p50=%u p95=%u p99=%u degree_eq_R_frac=%.6f "
              "compatible_avg=%.3f compatible_p50=%u compatible_p95=%u compatible_p99=%u "
              "min_per_label_avg=%.3f min_per_label_p50=%u min_per_label_p95=%u min_per_label_p99=%u "
              "diagnostic_seconds=%.6f\n",
              deg_sum / n, pd[0], pd[1], pd[2], at_R / n, compat_sum / n, pc[0], pc[1], pc[2], minpl_sum / n, pm[0],
              pm[1], pm[2], now_sec() - t0);
  std::fflush(stdout);
  return 0;
}

// Processing order of the rows (row kernels) and of the per-label tasks:
// rows sorted by their three nearest of K evenly spaced pivot rows (the
// standard build's locality schedule, K from DANCE_LOCALITY_CELLS, default
// 1024, 0: identity order; c5 814 -> 810 ms against the nearest pivot alone),
// and each row's tasks in that row order. Waves in flight then work
// on neighbouring rows, whose searches share rows in L2. Results do not depend
// on the order. Scratch: lsort / lrows (sort), roff (task offsets).
// Target entries of a long-list prune key window (k_csr_long):
// DANCE_LONG_WINDOW, default 2048, clamped to 64 .. kLongList / 2. Results do
// not depend on it.
static uint32_t long_window() {
  const char* e = std::getenv("DANCE_LONG_WINDOW");
  const uint32_t v = e && e[0] ? (uint32_t)std::strtoul(e, nullptr, 10) : 2048u;
  return std::min(std::max(v, 64u), kLongList / 2u);
}

int locality_order(const Rows& rows, const Labels& Ld, uint32_t N, uint32_t T, FState& st, ScanWorkspace& scan,
                   SortWorkspace& sort_ws, hipStream_t s, const uint32_t** rorder, const uint32_t** torder) {
  const char* e = std::getenv("DANCE_LOCALITY_CELLS");
  const uint32_t K = std::min(e && e[0] ? (uint32_t)std::strtoul(e, nullptr, 10) : 1024u, N);
  *rorder = *torder = nullptr;
  if (K < 2) return 0;
  DevBuf piv;
  DCHECK(piv.alloc((size_t)K * 4));
  hipLaunchKernelGGL(k_pivots, dim3((K + 255) / 256), dim3(256), 0, s, N, K, piv.as<uint32_t>());
  DHIP(hipGetLastError());
  uint32_t* kb[2] = {st.lsort.as<uint32_t>(), st.lsort.as<uint32_t>() + N};
  uint32_t* vb[2] = {st.lrows.as<uint32_t>(), st.lsort.as<uint32_t>() + 2 * (size_t)N};
  DCHECK(with_dt_cpl(rows.dtype, pick_cpl(rows.rs.nch), [&](auto dt, auto c) {
    hipLaunchKernelGGL((k_cells<decltype(dt)::value, decltype(c)::value>), dim3(cells_grid(N)), dim3(kCellsBlock), 0,
                       s, rows.rs, N, piv.as<const uint32_t>(), K, cell_levels(K, 3), kb[0], vb[0]);
    DHIP(hipGetLastError());
    return 0;
  }));
  int which = 0;
  const uint64_t nkeys = cell_levels(K, 3) == 3u ? (uint64_t)K * K * K : (uint64_t)K;
  DCHECK(radix_sort_pairs(kb, vb, N, bit_length((uint32_t)(nkeys - 1)), sort_ws, s, &which));
  DCHECK(st.rorder.alloc((size_t)N * 4));
  DHIP(hipMemcpyAsync(st.rorder.p, vb[which], (size_t)N * 4, hipMemcpyDeviceToDevice, s));
  if (T) {
    uint32_t* pos = st.roff.as<uint32_t>();  // N + 1 entries, free until the rounds
    DCHECK(st.torder.alloc((size_t)T * 4));
    hipLaunchKernelGGL(k_task_counts, dim3(grid_thr((uint64_t)N + 1)), dim3(256), 0, s, N, Ld.off,
                       st.rorder.as<const uint32_t>(), pos);
    DHIP(hipGetLastError());
    DCHECK(scan_exclusive(pos, (size_t)N + 1, scan, s));
    hipLaunchKernelGGL(k_task_fill, dim3(grid_thr(N)), dim3(256), 0, s, N, Ld.off, st.rorder.as<const uint32_t>(),
                       pos, st.torder.as<uint32_t>());
    DHIP(hipGetLastError());
    *torder = st.torder.as<const uint32_t>();
  }
  *rorder = st.rorder.as<const uint32_t>();
  return 0;
}

// Runs the build on resident rows; on success st.ga / st.da hold the graph.
int run_filtered(const Rows& rows, const FParams& p, const uint32_t* h_off, const uint32_t* h_lab,
                 const uint32_t* h_starts, hipStream_t s, FState& st, GPUFilteredVamanaStats& gs,
                 DanceFilteredProfile& kp) {
  const uint32_t N = p.N, R = p.R, T = p.total;
  const uint32_t work_C = std::min(p.C, kMaxWorkC);
  const int cpl = pick_cpl(rows.rs.nch);
  if (cpl < 0) {
    std::fprintf(stderr, "%s dim=%u is beyond the supported row width\n", kTag, p.dim);
    return -1;
  }
  if ((uint64_t)N * R > 0xFFFFFFFFull) {
    std::fprintf(stderr, "%s N*R=%llu exceeds 2^32 edges\n", kTag, (unsigned long long)N * R);
    return -1;
  }
  const uint32_t per_label_pool = std::min(p.filtered_L, 32u), per_label_keep = std::min(per_label_pool, 8u);
  const uint32_t ordinary_keep = std::min(R, p.L), ordinary_pool = std::min(64u, p.filtered_L);

  // Label -> points postings, ascending rows (:5768-5800).
  const uint32_t nl = std::max(1u, p.num_labels);
  const double tl = now_sec();
  std::vector<uint32_t> lpo((size_t)nl + 1, 0);
  for (uint32_t i = 0; i < T; ++i)
    if (h_lab[i] < p.num_labels) ++lpo[(size_t)h_lab[i] + 1];
  for (uint32_t l = 0; l < p.num_labels; ++l) lpo[l + 1] += lpo[l];
  std::vector<uint32_t> lpts(std::max<size_t>(1, lpo[p.num_labels]), DANCE_INV);
  {
    std::vector<uint32_t> cur(lpo.begin(), lpo.end());
    for (uint32_t r = 0; r < N; ++r)
      for (uint32_t i = h_off[r]; i < h_off[r + 1]; ++i)
        if (h_lab[i] < p.num_labels) lpts[cur[h_lab[i]]++] = r;
  }
  DCHECK(st.off.alloc((size_t)(N + 1) * 4));
  DCHECK(st.lab.alloc((size_t)std::max(1u, T) * 4));
  DCHECK(st.lpo.alloc(lpo.size() * 4));
  DCHECK(st.lpts.alloc(lpts.size() * 4));
  DCHECK(st.starts.alloc((size_t)nl * 4));
  DCHECK(st.task_rows.alloc((size_t)std::max(1u, T) * 4));

  DHIP(hipMemcpyAsync(st.off.p, h_off, (size_t)(N + 1) * 4, hipMemcpyHostToDevice, s));
  if (T) DHIP(hipMemcpyAsync(st.lab.p, h_lab, (size_t)T * 4, hipMemcpyHostToDevice, s));
  DHIP(hipMemcpyAsync(st.lpo.p, lpo.data(), lpo.size() * 4, hipMemcpyHostToDevice, s));
  DHIP(hipMemcpyAsync(st.lpts.p, lpts.data(), lpts.size() * 4, hipMemcpyHostToDevice, s));
  DHIP(hipMemcpyAsync(st.starts.p, h_starts, (size_t)nl * 4, hipMemcpyHostToDevice, s));
  DHIP(hipStreamSynchronize(s));
  gs.label_h2d_seconds = now_sec() - tl;

  const size_t NR = (size_t)N * R;
  DCHECK(st.ga.alloc(NR * 4));
  DCHECK(st.gb.alloc(NR * 4));
  DCHECK(st.da.alloc((size_t)N * 4));
  DCHECK(st.db.alloc((size_t)N * 4));
  DCHECK(st.tids.alloc((size_t)std::max(1u, T) * std::max(1u, per_label_keep) * 4));
  DCHECK(st.td.alloc((size_t)std::max(1u, T) * std::max(1u, per_label_keep) * 4));
  DCHECK(st.roff.alloc((size_t)(N + 1) * 4));
  DCHECK(st.cursor.alloc((size_t)N * 4));
  DCHECK(st.rids.alloc(std::max<size_t>(1, NR) * 4));
  DCHECK(st.boff.alloc((size_t)(N + 1) * 4));
  DCHECK(st.lrows.alloc((size_t)N * 4));
  DCHECK(st.lsort.alloc((size_t)N * 12));  // keys (2 buffers) + a second value buffer
  DCHECK(st.lcount.alloc(8));  // long rows, rows beyond the key window
  DCHECK(st.ctr.alloc((size_t)kCtrStripes * kNumCounters * 8));
  DCHECK(st.d32.alloc(8 * 4));
  DCHECK(st.d64.alloc(8 * 8));
  DHIP(hipMemsetAsync(st.ctr.p, 0, (size_t)kCtrStripes * kNumCounters * 8, s));
  unsigned long long* ctr = st.ctr.as<unsigned long long>();
  ScanWorkspace scan;
  SortWorkspace sort_ws;

  // Fixed-width label rows for membership tests (DANCE_FILTERED_LAB8=0: list
  // walks only), and per-point label signatures carried next to the round's
  // input graph so the searches reject most neighbours without a label read
  // (DANCE_FILTERED_SIG=0: off). Neither changes a result.
  const char* l8e = std::getenv("DANCE_FILTERED_LAB8");
  const bool use_lab8 = !(l8e && l8e[0] == '0');
  const char* sge = std::getenv("DANCE_FILTERED_SIG");
  const bool use_sig = !(sge && sge[0] == '0');
  if (use_lab8) DCHECK(st.lab8.alloc((size_t)N * 32));
  DCHECK(st.sig.alloc((size_t)N * 4));
  if (use_sig && p.rounds) DCHECK(st.gsig.alloc(NR * 4));
  hipLaunchKernelGGL(k_lab8, dim3(grid_thr(N)), dim3(256), 0, s, N, st.off.as<uint32_t>(), st.lab.as<uint32_t>(),
                     use_lab8 ? st.lab8.as<uint4>() : nullptr, st.sig.as<uint32_t>());
  DHIP(hipGetLastError());
  Labels Ld{st.off.as<uint32_t>(), st.lab.as<uint32_t>(), st.lpo.as<uint32_t>(), st.lpts.as<uint32_t>(),
            st.starts.as<uint32_t>(), p.num_labels, p.universal, use_lab8 ? st.lab8.as<const uint4>() : nullptr,
            use_sig ? st.sig.as<const uint32_t>() : nullptr};
  uint32_t* ga = st.ga.as<uint32_t>();
  uint32_t* gb = st.gb.as<uint32_t>();
  uint32_t* da = st.da.as<uint32_t>();
  uint32_t* db = st.db.as<uint32_t>();
  uint32_t* roff = st.roff.as<uint32_t>();
  uint32_t* boff = st.boff.as<uint32_t>();

  FEvents E;
  // Rows of more than kCsrRegMax candidates (label hubs) are pruned on a
  // second stream, concurrently with the short rows: the largest hub holds
  // one workgroup for tens of ms, which the short rows' kernel then hides.
  StreamGuard s2g, s3g;
  DHIP(hipStreamCreate(&s2g.s));
  DHIP(hipStreamCreate(&s3g.s));
  const hipStream_t s2 = s2g.s, s3 = s3g.s;
  hipEvent_t e0 = E.mark(s);
  hipLaunchKernelGGL(k_random_graph, dim3(grid_thr(N)), dim3(256), 0, s, N, R,
                     std::min(std::min(kBackboneDegree, R), N - 1), kBackboneSeed, ga, da);
  DHIP(hipGetLastError());
  hipEvent_t e1 = E.mark(s);
  hipLaunchKernelGGL(k_task_rows, dim3(grid_thr(N)), dim3(256), 0, s, N, Ld.off, st.task_rows.as<uint32_t>());
  DHIP(hipGetLastError());
  const uint32_t* rorder = nullptr;
  const uint32_t* torder = nullptr;
  DCHECK(locality_order(rows, Ld, N, T, st, scan, sort_ws, s, &rorder, &torder));
  hipEvent_t e2 = E.mark(s);
  kp.backbone_ms = ms_between(e0, e1);
  double task_ms = 0, row_ms = 0, rev_ms = 0, csr_ms = 0;
  const size_t search_lds = (size_t)kWaves * kSearchLds * 4;
  const size_t csr_lds = (size_t)kWaves * kCsrLds * 4;
  uint64_t reverse_edges = 0;
  const bool log = filtered_log();
  if (log) {
    // The knobs behind the fixed values are the reference's defaults
    // (:5689-5700): no round-0 ordinary search variants, no posting or round-0
    // anchors, the bridge reserve (used only by the true-ordinary round 0),
    // no active frontier.
    std::printf("[gpu_vamana_filtered_navigation_policy] per_label_pool=%u per_label_keep=%u "
                "true_ordinary_round0=0 pure_ordinary_round0=0 ordinary_pool=%u ordinary_steps=32 "
                "posting_anchor=0 additional_round0_anchor=0 bridge_work_reserve=8 active_frontier=0 "
                "label_quota=1 exact_csr_reverse=1\n",
                per_label_pool, per_label_keep, ordinary_pool);
    if (p.rounds) {
      DCHECK(st.prev_g.alloc(NR * 4));
      DCHECK(st.prev_d.alloc((size_t)N * 4));
      DCHECK(st.rcnt.alloc(2 * 8));
    }
  }

  for (uint32_t round = 0; round < p.rounds; ++round) {
    Graph Ga{N, R, ga, da};
    if (use_sig) {
      hipLaunchKernelGGL(k_graph_sig, grid_dims((NR + 255) / 256, 256), dim3(256), 0, s, N, R, static_cast<const uint32_t*>(ga),
                         static_cast<const uint32_t*>(da), st.sig.as<const uint32_t>(), st.gsig.as<uint32_t>());
      DHIP(hipGetLastError());
      Ga.sig = st.gsig.as<const uint32_t>();
    }
    if (log) {
      DHIP(hipMemcpyAsync(st.prev_g.p, ga, NR * 4, hipMemcpyDeviceToDevice, s));
      DHIP(hipMemcpyAsync(st.prev_d.p, da, (size_t)N * 4, hipMemcpyDeviceToDevice, s));
    }
    hipEvent_t r0 = E.mark(s);
    if (T > 0) {
      DCHECK(with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
        hipLaunchKernelGGL((k_task_search<decltype(dt)::value, decltype(c)::value>), grid_xcd(T),
                           dim3(kBlock), search_lds, s, rows.rs, Ga, Ld, st.task_rows.as<const uint32_t>(), torder,
                           T, per_label_pool, per_label_keep, p.STEPS, st.tids.as<uint32_t>(), st.td.as<float>(),
                           ctr);
        DHIP(hipGetLastError());
        return 0;
      }));
    }
    hipEvent_t r1 = E.mark(s);
    RowArgs A{ordinary_pool, ordinary_keep, p.STEPS, p.global_start, work_C, per_label_keep, p.alpha,
              st.tids.as<const uint32_t>(), st.td.as<const float>(), gb, db, ctr, rorder};
    DCHECK(with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
      hipLaunchKernelGGL((k_row<decltype(dt)::value, decltype(c)::value>), grid_xcd(N), dim3(kBlock),
                         search_lds, s, rows.rs, Ga, Ld, A);
      DHIP(hipGetLastError());
      return 0;
    }));
    hipEvent_t r2 = E.mark(s);
    // exact reverse CSR of the forward graph
    DHIP(hipMemsetAsync(roff, 0, (size_t)(N + 1) * 4, s));
    hipLaunchKernelGGL(k_rev_count, dim3(grid_thr(N)), dim3(256), 0, s, N, R, gb, db, roff);
    DHIP(hipGetLastError());
    DCHECK(scan_exclusive(roff, (size_t)N + 1, scan, s));
    DHIP(hipMemsetAsync(st.cursor.p, 0, (size_t)N * 4, s));
    hipLaunchKernelGGL(k_rev_fill, dim3(grid_thr(N)), dim3(256), 0, s, N, R, gb, db, roff,
                       st.cursor.as<uint32_t>(), st.rids.as<uint32_t>());
    DHIP(hipGetLastError());
    hipLaunchKernelGGL(k_big_sizes, dim3(grid_thr((uint64_t)N + 1)), dim3(256), 0, s, N, R, db, roff, boff);
    DHIP(hipGetLastError());
    DCHECK(scan_exclusive(boff, (size_t)N + 1, scan, s));
    DHIP(hipMemsetAsync(st.lcount.p, 0, 8, s));
    const uint32_t win = long_window();
    uint32_t* lkeys[2] = {st.lsort.as<uint32_t>(), st.lsort.as<uint32_t>() + N};
    uint32_t* lvals[2] = {st.lrows.as<uint32_t>(), st.lsort.as<uint32_t>() + 2 * (size_t)N};
    hipLaunchKernelGGL(k_long_rows, dim3(grid_thr(N)), dim3(256), 0, s, N, boff, win, lvals[0], lkeys[0],
                       st.lcount.as<uint32_t>());
    DHIP(hipGetLastError());
    uint32_t tails[4] = {0, 0, 0, 0};
    DHIP(hipMemcpyAsync(&tails[0], roff + N, 4, hipMemcpyDeviceToHost, s));
    DHIP(hipMemcpyAsync(&tails[1], boff + N, 4, hipMemcpyDeviceToHost, s));
    DHIP(hipMemcpyAsync(&tails[2], st.lcount.p, 8, hipMemcpyDeviceToHost, s));
    DHIP(hipStreamSynchronize(s));
    reverse_edges += tails[0];
    DCHECK(ensure_big(st, tails[1]));
    int lr = 0;  // long rows, longest first
    if (tails[2] > 1) DCHECK(radix_sort_pairs(lkeys, lvals, tails[2], 32, sort_ws, s, &lr));
    hipEvent_t r3 = E.mark(s);
    const Graph Gb{N, R, gb, db};
    CsrArgs Cs{p.alpha, roff, st.rids.as<const uint32_t>(), boff, st.bd.as<float>(), st.brem.as<uint8_t>(),
               st.bmask.as<uint32_t>(), ga, da, ctr, win};
    DCHECK(with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
      // The three kernels write disjoint rows and run side by side: long
      // rows beyond the key window (the first tails[3] of the longest-first
      // list; workgroups of kLongWaves waves), the other long rows
      // (kLongSmallWaves), and k_csr for the short lists.
      hipEvent_t long_done = nullptr, hub_done = nullptr;
      const uint32_t hubs = tails[3], rest = tails[2] - tails[3];
      if (hubs > 0) {
        DHIP(hipStreamWaitEvent(s3, r3, 0));
        hipLaunchKernelGGL((k_csr_long<decltype(dt)::value, decltype(c)::value, (int)kLongWaves>), dim3(hubs),
                           dim3(kLongBlock), 0, s3, rows.rs, Gb, Ld, Cs, lvals[lr]);
        DHIP(hipGetLastError());
        hub_done = E.mark(s3);
        if (!hub_done) return -1;
      }
      if (rest > 0) {
        DHIP(hipStreamWaitEvent(s2, r3, 0));
        hipLaunchKernelGGL((k_csr_long<decltype(dt)::value, decltype(c)::value, (int)kLongSmallWaves>), dim3(rest),
                           dim3(64u * kLongSmallWaves), 0, s2, rows.rs, Gb, Ld, Cs, lvals[lr] + hubs);
        DHIP(hipGetLastError());
        long_done = E.mark(s2);
        if (!long_done) return -1;
      }
      hipLaunchKernelGGL((k_csr<decltype(dt)::value, decltype(c)::value>), grid_xcd(N), dim3(kBlock), csr_lds,
                         s, rows.rs, Gb, Ld, Cs);
      DHIP(hipGetLastError());
      if (long_done) DHIP(hipStreamWaitEvent(s, long_done, 0));
      if (hub_done) DHIP(hipStreamWaitEvent(s, hub_done, 0));
      return 0;
    }));
    hipEvent_t r4 = E.mark(s);
    DHIP(hipEventSynchronize(r4));
    task_ms += ms_between(r0, r1);
    row_ms += ms_between(r1, r2);
    rev_ms += ms_between(r2, r3);
    csr_ms += ms_between(r3, r4);
    peak_mem(gs.peak_gpu_mem_gb);
    if (log) {
      unsigned long long rc[2] = {0, 0};
      DHIP(hipMemsetAsync(st.rcnt.p, 0, sizeof(rc), s));
      hipLaunchKernelGGL(k_round_changes, dim3((N + 3) / 4), dim3(256), 0, s, N, R, st.prev_g.as<const uint32_t>(),
                         st.prev_d.as<const uint32_t>(), static_cast<const uint32_t*>(ga),
                         static_cast<const uint32_t*>(da), static_cast<const uint32_t*>(roff),
                         st.rcnt.as<unsigned long long>());
      DHIP(hipGetLastError());
      DHIP(hipMemcpyAsync(rc, st.rcnt.p, sizeof(rc), hipMemcpyDeviceToHost, s));
      DHIP(hipStreamSynchronize(s));
      std::printf("[gpu_vamana_filtered_canonical_round] round=%u kind=full alpha=%.3f active=%u tasks=%u "
                  "changed=%llu touched=%llu reverse_proposals=%u deficient=0 next_active=%u\n",
                  round, p.alpha, N, T, rc[0], rc[1], tails[0], N);
    }
  }
  if (log) std::printf("[gpu_vamana_filtered_label_coverage_repair] disabled=1\n");
  if (p.rounds == 0) DHIP(hipStreamSynchronize(s));

  // publish step (gpu_vamana_filtered.cu:6328-6432)
  const uint32_t PR = publish_degree(R);
  st.out_R = R;
  st.out_g = ga;
  st.out_d = da;
  uint32_t pub_tail = 0;
  double pub_ms = 0;
  if (PR < R) {
    const size_t pub_lds = (size_t)kWaves * kPubLds * 4;
    hipEvent_t p0 = E.mark(s);
    PubArgs P{p.alpha, PR, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, gb, db, ctr};
    DCHECK(with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
      hipLaunchKernelGGL((k_publish<decltype(dt)::value, decltype(c)::value, false>), grid_xcd(N),
                         dim3(kBlock), pub_lds, s, rows.rs, Graph{N, R, ga, da}, Ld, P);
      DHIP(hipGetLastError());
      return 0;
    }));
    DHIP(hipMemsetAsync(roff, 0, (size_t)(N + 1) * 4, s));
    hipLaunchKernelGGL(k_rev_count, dim3(grid_thr(N)), dim3(256), 0, s, N, PR, gb, db, roff);
    DHIP(hipGetLastError());
    DCHECK(scan_exclusive(roff, (size_t)N + 1, scan, s));
    DHIP(hipMemsetAsync(st.cursor.p, 0, (size_t)N * 4, s));
    hipLaunchKernelGGL(k_rev_fill, dim3(grid_thr(N)), dim3(256), 0, s, N, PR, gb, db, roff,
                       st.cursor.as<uint32_t>(), st.rids.as<uint32_t>());
    DHIP(hipGetLastError());
    hipLaunchKernelGGL(k_big_sizes, dim3(grid_thr((uint64_t)N + 1)), dim3(256), 0, s, N, PR, db, roff, boff);
    DHIP(hipGetLastError());
    DCHECK(scan_exclusive(boff, (size_t)N + 1, scan, s));
    uint32_t tails[2] = {0, 0};
    DHIP(hipMemcpyAsync(&tails[0], roff + N, 4, hipMemcpyDeviceToHost, s));
    DHIP(hipMemcpyAsync(&tails[1], boff + N, 4, hipMemcpyDeviceToHost, s));
    DHIP(hipStreamSynchronize(s));
    pub_tail = tails[1];
    DCHECK(ensure_big(st, tails[1]));
    P = PubArgs{p.alpha, PR, roff, st.rids.as<const uint32_t>(), boff, st.bmask.as<uint32_t>(), st.bd.as<float>(),
                st.brem.as<uint8_t>(), gb, db, ctr};
    DCHECK(with_dt_cpl(rows.dtype, cpl, [&](auto dt, auto c) {
      hipLaunchKernelGGL((k_publish<decltype(dt)::value, decltype(c)::value, true>), grid_xcd(N),
                         dim3(kBlock), pub_lds, s, rows.rs, Graph{N, PR, gb, db}, Ld, P);
      DHIP(hipGetLastError());
      return 0;
    }));
    hipEvent_t p1 = E.mark(s);
    DHIP(hipEventSynchronize(p1));
    pub_ms = ms_between(p0, p1);
    st.out_R = PR;
    st.out_g = gb;
    st.out_d = db;
    peak_mem(gs.peak_gpu_mem_gb);
  }

  // diagnostics of the final graph
  hipEvent_t g0 = E.mark(s);
  const uint32_t init32[8] = {0, 0, 0, 0xFFFFFFFFu, 0, 0xFFFFFFFFu, 0, 0};
  DHIP(hipMemcpyAsync(st.d32.p, init32, sizeof(init32), hipMemcpyHostToDevice, s));
  DHIP(hipMemsetAsync(st.d64.p, 0, 8 * 8, s));
  hipLaunchKernelGGL(k_diagnostics, dim3(grid_thr(N)), dim3(256), 0, s,
                     Graph{N, st.out_R, static_cast<const uint32_t*>(st.out_g), static_cast<const uint32_t*>(st.out_d)}, Ld,
                     st.d32.as<uint32_t>(), st.d64.as<unsigned long long>());
  DHIP(hipGetLastError());
  hipEvent_t g1 = E.mark(s);
  uint32_t h32[8];
  unsigned long long h64[8], hc[kNumCounters] = {};
  std::vector<unsigned long long> stripes((size_t)kCtrStripes * kNumCounters);
  DHIP(hipMemcpyAsync(h32, st.d32.p, sizeof(h32), hipMemcpyDeviceToHost, s));
  DHIP(hipMemcpyAsync(h64, st.d64.p, sizeof(h64), hipMemcpyDeviceToHost, s));
  DHIP(hipMemcpyAsync(stripes.data(), st.ctr.p, stripes.size() * 8, hipMemcpyDeviceToHost, s));
  DHIP(hipStreamSynchronize(s));
  for (size_t i = 0; i < stripes.size(); ++i) {
    const size_t k = i % kNumCounters;
    hc[k] = k == kBigMax ? std::max(hc[k], stripes[i]) : hc[k] + stripes[i];
  }

  // Published stats follow the reference's release path (:8648-8718): search
  // counters are reported as zero there and the candidate counts are the
  // final edge counts; the device counters go to DanceFilteredProfile.
  gs.backbone_seconds = kp.backbone_ms * 1e-3;
  gs.graph_build_seconds = gs.backbone_seconds;
  gs.task_generation_seconds = ms_between(e1, e2) * 1e-3;
  gs.filtered_search_seconds = task_ms * 1e-3;
  gs.ordinary_search_seconds = row_ms * 1e-3;
  gs.csr_reverse_seconds = rev_ms * 1e-3;
  gs.reverse_prune_seconds = csr_ms * 1e-3;
  gs.diagnostics_seconds = ms_between(g0, g1) * 1e-3;
  gs.invalid_neighbor_count = h32[0];
  gs.self_loop_count = h32[1];
  gs.low_common_label_degree_count = h32[2];
  gs.out_degree_min = h32[3];
  gs.out_degree_max = h32[4];
  gs.common_label_degree_min = h32[5];
  gs.common_label_degree_max = h32[6];
  gs.out_degree_avg = (double)h64[0] / N;
  gs.avg_common_label_out_degree = (double)h64[1] / N;
  gs.label_check_count = h64[2];
  gs.label_reject_count = h64[3];
  gs.universal_label_pass_count = h64[4];
  gs.filtered_candidate_count = h64[1];
  gs.unfiltered_candidate_count = h64[0];
  gs.merged_candidate_count = h64[0];
  gs.final_prune_rows = N;
  gs.semantic_stage = kStageLabelSync;
  gs.semantic_complete = 1;
  if (log) DCHECK(print_degree_profile(st, Ld, N, s));
  peak_mem(gs.peak_gpu_mem_gb);

  kp.rounds = p.rounds;
  kp.vector_bytes = rows.vbytes();
  kp.task_search_ms = task_ms;
  kp.row_ms = row_ms;
  kp.reverse_ms = rev_ms;
  kp.csr_ms = csr_ms;
  kp.diagnostics_ms = ms_between(g0, g1);
  kp.total_ms = ms_between(e0, g1);
  kp.task_dist = hc[kTaskDist];
  kp.union_dist = hc[kUnionDist];
  kp.work_dist = hc[kWorkDist];
  kp.prune_dist = hc[kPruneDist];
  kp.csr_dist = hc[kCsrDist];
  kp.csr_prune_dist = hc[kCsrPruneDist];
  kp.merged_candidates = hc[kMergedCands];
  kp.quota_dropped = hc[kQuotaDropped];
  kp.reverse_edges = reverse_edges;
  kp.touched_rows = hc[kTouchedRows];
  kp.csr_candidates = hc[kCsrCandidates];
  kp.long_lists = hc[kBigRows];
  kp.long_max_candidates = hc[kBigMax];
  kp.publish_ms = pub_ms;
  kp.publish_dist = hc[kPubDist];
  kp.publish_touched = hc[kPubTouched];
  kp.task_expansions = hc[kTaskExp];
  kp.task_label_reads = hc[kTaskLab];
  kp.union_expansions = hc[kUnionExp];
  kp.union_label_reads = hc[kUnionLab];
  kp.publish_long_entries = pub_tail;
  kp.publish_degree = st.out_R;
  kp.out_edges = h64[0];
  kp.common_edges = h64[1];
  if (verbose())
    std::printf("%s N=%u dim=%u R=%u L=%u FilteredL=%u C=%u labels=%u total=%u rounds=%u total_ms=%.3f\n", kTag, N,
                p.dim, R, p.L, p.filtered_L, p.C, p.num_labels, T, p.rounds, kp.total_ms);
  return 0;
}

// Host-input build. src_dtype: DANCE_F32 (searched as fp16), DANCE_U8 or
// DANCE_F16 (host fp16 rows, used by tests).
int filtered_host(const void* h_data, int src_dtype, const FParams& p, const uint32_t* off, const uint32_t* lab,
                  const uint32_t* starts, uint32_t* h_graph, uint32_t* h_degree) {
  std::lock_guard<std::mutex> lk(g_fmu);
  g_fstats = GPUFilteredVamanaStats{};
  g_fprof = DanceFilteredProfile{};
  const double t0 = now_sec();
  if (!h_data || !h_graph || !h_degree) {
    std::fprintf(stderr, "%s null input pointer.\n", kTag);
    return -1;
  }
  if (const int rc = validate(p, off, lab, starts)) return rc;
  StreamGuard sg;
  DHIP(hipStreamCreate(&sg.s));
  hipStream_t s = sg.s;
  const int store = src_dtype == DANCE_U8 ? DANCE_U8 : DANCE_F16;
  Rows rows;
  DCHECK(setup_rows(rows, h_data, false, src_dtype, store, p.N, p.dim, s));
  DHIP(hipStreamSynchronize(s));
  GPUFilteredVamanaStats gs{};
  DanceFilteredProfile kp{};
  FState st;
  const int rc = run_filtered(rows, p, off, lab, starts, s, st, gs, kp);
  if (rc != 0) return rc;
  const double td = now_sec();
  DHIP(hipDeviceSynchronize());  // every build stream; the staged copies run on streams of their own
  DCHECK(copy_pageable(h_graph, st.out_g, (size_t)p.N * st.out_R * 4, hipMemcpyDeviceToHost));
  DCHECK(copy_pageable(h_degree, st.out_d, (size_t)p.N * 4, hipMemcpyDeviceToHost));
  gs.d2h_seconds = now_sec() - td;
  gs.gpu_build_seconds = now_sec() - t0;
  g_fstats = gs;
  g_fprof = kp;
  return 0;
}

FParams make_params(uint32_t N, uint32_t dim, uint32_t R, uint32_t L, uint32_t filtered_L, uint32_t C,
                    uint32_t STEPS, float alpha, uint32_t total, uint32_t num_labels, uint32_t universal,
                    uint32_t global_start, uint32_t rounds) {
  return FParams{N, dim, R, L, filtered_L, C, STEPS, alpha, total, num_labels, universal, global_start, rounds};
}

}  // namespace
}  // namespace dance

using namespace dance;

extern "C" {

int gpu_vamana_filtered_build_uint8(const uint8_t* h_data, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t L,
                                    uint32_t filtered_L, uint32_t C, uint32_t STEPS, float alpha,
                                    const uint32_t* point_label_offsets, const uint32_t* point_labels,
                                    uint32_t total_label_count, const uint32_t* label_to_start_id,
                                    uint32_t num_labels, uint32_t universal_label_id, uint32_t global_start_id,
                                    const uint32_t* query_anchor_offsets, const uint32_t* query_anchor_ids,
                                    uint32_t query_anchor_count, uint32_t* h_graph, uint32_t* h_degree) {
  (void)query_anchor_offsets;
  (void)query_anchor_ids;
  (void)query_anchor_count;
  return filtered_host(h_data, DANCE_U8,
                       make_params(num_points, dim, R, L, filtered_L, C, STEPS, alpha, total_label_count, num_labels,
                                   universal_label_id, global_start_id, kRounds),
                       point_label_offsets, point_labels, label_to_start_id, h_graph, h_degree);
}

int gpu_vamana_filtered_build_float(const float* h_data, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t L,
                                    uint32_t filtered_L, uint32_t C, uint32_t STEPS, float alpha,
                                    const uint32_t* point_label_offsets, const uint32_t* point_labels,
                                    uint32_t total_label_count, const uint32_t* label_to_start_id,
                                    uint32_t num_labels, uint32_t universal_label_id, uint32_t global_start_id,
                                    const uint32_t* query_anchor_offsets, const uint32_t* query_anchor_ids,
                                    uint32_t query_anchor_count, uint32_t* h_graph, uint32_t* h_degree) {
  (void)query_anchor_offsets;
  (void)query_anchor_ids;
  (void)query_anchor_count;
  return filtered_host(h_data, DANCE_F32,
                       make_params(num_points, dim, R, L, filtered_L, C, STEPS, alpha, total_label_count, num_labels,
                                   universal_label_id, global_start_id, kRounds),
                       point_label_offsets, point_labels, label_to_start_id, h_graph, h_degree);
}

void gpu_vamana_filtered_get_last_stats(GPUFilteredVamanaStats* stats) {
  if (!stats) return;
  std::lock_guard<std::mutex> lk(g_fmu);
  *stats = g_fstats;
}

int dance_filtered_build(const void* h_data, int dtype, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t L,
                         uint32_t filtered_L, uint32_t C, uint32_t STEPS, float alpha,
                         const uint32_t* point_label_offsets, const uint32_t* point_labels,
                         uint32_t total_label_count, const uint32_t* label_to_start_id, uint32_t num_labels,
                         uint32_t universal_label_id, uint32_t global_start_id, uint32_t rounds, uint32_t* h_graph,
                         uint32_t* h_degree) {
  if (dtype != DANCE_F32 && dtype != DANCE_U8 && dtype != DANCE_F16) {
    std::fprintf(stderr, "[gpu_vamana_filtered] unsupported dtype %d\n", dtype);
    return -1;
  }
  return filtered_host(h_data, dtype,
                       make_params(num_points, dim, R, L, filtered_L, C, STEPS, alpha, total_label_count, num_labels,
                                   universal_label_id, global_start_id, rounds),
                       point_label_offsets, point_labels, label_to_start_id, h_graph, h_degree);
}

int dance_filtered_build_resident(const void* d_data, int dtype, uint32_t num_points, uint32_t dim, uint32_t R,
                                  uint32_t L, uint32_t filtered_L, uint32_t C, uint32_t STEPS, float alpha,
                                  const uint32_t* point_label_offsets, const uint32_t* point_labels,
                                  uint32_t total_label_count, const uint32_t* label_to_start_id,
                                  uint32_t num_labels, uint32_t universal_label_id, uint32_t global_start_id,
                                  uint32_t* d_graph, uint32_t* d_degree) {
  std::lock_guard<std::mutex> lk(g_fmu);
  g_fstats = GPUFilteredVamanaStats{};
  g_fprof = DanceFilteredProfile{};
  const double t0 = now_sec();
  if (!d_data || !d_graph || !d_degree) {
    std::fprintf(stderr, "[gpu_vamana_filtered] null input pointer.\n");
    return -1;
  }
  if (dtype != DANCE_F32 && dtype != DANCE_U8 && dtype != DANCE_F16) {
    std::fprintf(stderr, "[gpu_vamana_filtered] unsupported dtype %d\n", dtype);
    return -1;
  }
  const FParams p = make_params(num_points, dim, R, L, filtered_L, C, STEPS, alpha, total_label_count, num_labels,
                                universal_label_id, global_start_id, kRounds);
  if (const int rc = validate(p, point_label_offsets, point_labels, label_to_start_id)) return rc;
  StreamGuard sg;
  DHIP(hipStreamCreate(&sg.s));
  hipStream_t s = sg.s;
  Rows rows;
  DCHECK(setup_rows(rows, d_data, true, dtype, dtype == DANCE_U8 ? DANCE_U8 : DANCE_F16, p.N, p.dim, s));
  GPUFilteredVamanaStats gs{};
  DanceFilteredProfile kp{};
  FState st;
  const int rc = run_filtered(rows, p, point_label_offsets, point_labels, label_to_start_id, s, st, gs, kp);
  if (rc != 0) return rc;
  DHIP(hipMemcpyAsync(d_graph, st.out_g, (size_t)p.N * st.out_R * 4, hipMemcpyDeviceToDevice, s));
  DHIP(hipMemcpyAsync(d_degree, st.out_d, (size_t)p.N * 4, hipMemcpyDeviceToDevice, s));
  DHIP(hipStreamSynchronize(s));
  gs.gpu_build_seconds = now_sec() - t0;
  g_fstats = gs;
  g_fprof = kp;
  return 0;
}

void dance_get_last_filtered_profile(DanceFilteredProfile* profile) {
  if (!profile) return;
  std::lock_guard<std::mutex> lk(g_fmu);
  *profile = g_fprof;
}

}  // extern "C"
