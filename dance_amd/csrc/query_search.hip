// Host side of the query search (dance_search / dance_search_resident in
// include/dance_hip.h): uploads what is not resident, launches k_query with
// the candidate-list width for L, and returns the k best ids and distances.
// Used by the recall measurement and by callers that want GPU search over a
// built graph (reference counterpart: DiskANN search_memory_index, filtered
// start points integrations/dance-diskann-78256bba.patch:20583-20600).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <mutex>

#include "../../include/dance_hip.h"
#include "host_common.h"
#include "query_kernels.h"

namespace dance {
namespace {

using namespace qs;

std::mutex g_qmu;
DanceSearchStats g_qstats{};

constexpr uint32_t kMaxL = 1024;  // 16 slots per lane
int pick_ps(uint32_t L) { return L <= 64 ? 1 : L <= 128 ? 2 : L <= 256 ? 4 : L <= 512 ? 8 : 16; }

struct SearchIn {
  const void* data;  // device rows (resident) or host rows
  bool data_on_device;
  int dtype;
  uint32_t N, dim;
  const uint32_t* graph;  // device (resident) or host
  const uint32_t* degree;
  bool graph_on_device;
  uint32_t R;
  const uint32_t* starts;
  uint32_t nstarts;
  const uint32_t* start_off;  // host, nq + 1 entries (nullptr: 1 shared or nq starts)
  const void* queries;  // host
  uint32_t nq, k, L;
  const uint32_t* label_offsets;  // host, optional
  const uint32_t* labels;
  const uint32_t* query_labels;
  uint32_t* ids_out;  // host
  float* d_out;
};

int run_search(const SearchIn& in) {
  if (!in.data || !in.graph || !in.degree || !in.starts || !in.queries || !in.ids_out || !in.d_out) {
    std::fprintf(stderr, "[dance_search] null input pointer.\n");
    return -1;
  }
  if (in.N == 0 || in.dim == 0 || in.R == 0 || in.nq == 0 || in.k == 0 || in.k > kMaxK || in.L < in.k ||
      in.L > kMaxL || (!in.start_off && in.nstarts != 1 && in.nstarts != in.nq)) {
    std::fprintf(stderr, "[dance_search] invalid parameters N=%u dim=%u R=%u nq=%u k=%u L=%u nstarts=%u\n", in.N,
                 in.dim, in.R, in.nq, in.k, in.L, in.nstarts);
    return -1;
  }
  if (in.start_off) {
    bool ok = in.start_off[0] == 0;
    for (uint32_t q = 0; ok && q < in.nq; ++q) ok = in.start_off[q] <= in.start_off[q + 1];
    if (!ok) {
      std::fprintf(stderr, "[dance_search] start_offsets must start at 0 and not decrease\n");
      return -1;
    }
  }
  const bool filt = in.label_offsets || in.labels || in.query_labels;
  if (filt && !(in.label_offsets && in.labels && in.query_labels)) {
    std::fprintf(stderr, "[dance_search] label filter needs offsets, labels and query labels\n");
    return -1;
  }
  if (in.dtype != DANCE_F32 && in.dtype != DANCE_U8 && in.dtype != DANCE_F16) {
    std::fprintf(stderr, "[dance_search] unsupported dtype %d\n", in.dtype);
    return -1;
  }
  std::lock_guard<std::mutex> lk(g_qmu);
  g_qstats = DanceSearchStats{};
  hipStream_t s = nullptr;
  DHIP(hipStreamCreate(&s));
  struct SG {
    hipStream_t s;
    ~SG() {
      if (s) (void)hipStreamDestroy(s);
    }
  } sg{s};
  Rows base, qr;
  DCHECK(setup_rows(base, in.data, in.data_on_device, in.dtype, in.dtype, in.N, in.dim, s));
  DCHECK(setup_rows(qr, in.queries, false, in.dtype, in.dtype, in.nq, in.dim, s));
  const int cpl = pick_cpl(base.rs.nch);
  if (cpl < 0) {
    std::fprintf(stderr, "[dance_search] dim=%u is beyond the supported row width\n", in.dim);
    return -1;
  }
  DevBuf g, dg, st, soff, off, lab, qlab, oi, od, ctr;
  const uint32_t* dgraph = in.graph;
  const uint32_t* ddeg = in.degree;
  if (!in.graph_on_device) {
    DCHECK(g.alloc((size_t)in.N * in.R * 4));
    DCHECK(dg.alloc((size_t)in.N * 4));
    DHIP(hipMemcpyAsync(g.p, in.graph, (size_t)in.N * in.R * 4, hipMemcpyHostToDevice, s));
    DHIP(hipMemcpyAsync(dg.p, in.degree, (size_t)in.N * 4, hipMemcpyHostToDevice, s));
    dgraph = g.as<uint32_t>();
    ddeg = dg.as<uint32_t>();
  }
  DCHECK(st.alloc((size_t)std::max(1u, in.nstarts) * 4));
  if (in.nstarts) DHIP(hipMemcpyAsync(st.p, in.starts, (size_t)in.nstarts * 4, hipMemcpyHostToDevice, s));
  if (in.start_off) {
    DCHECK(soff.alloc((size_t)(in.nq + 1) * 4));
    DHIP(hipMemcpyAsync(soff.p, in.start_off, (size_t)(in.nq + 1) * 4, hipMemcpyHostToDevice, s));
  }
  if (filt) {
    const uint32_t total = in.label_offsets[in.N];
    DCHECK(off.alloc((size_t)(in.N + 1) * 4));
    DCHECK(lab.alloc((size_t)std::max(1u, total) * 4));
    DCHECK(qlab.alloc((size_t)in.nq * 4));
    DHIP(hipMemcpyAsync(off.p, in.label_offsets, (size_t)(in.N + 1) * 4, hipMemcpyHostToDevice, s));
    if (total) DHIP(hipMemcpyAsync(lab.p, in.labels, (size_t)total * 4, hipMemcpyHostToDevice, s));
    DHIP(hipMemcpyAsync(qlab.p, in.query_labels, (size_t)in.nq * 4, hipMemcpyHostToDevice, s));
  }
  DCHECK(oi.alloc((size_t)in.nq * in.k * 4));
  DCHECK(od.alloc((size_t)in.nq * in.k * 4));
  DCHECK(ctr.alloc(3 * 8));
  DHIP(hipMemsetAsync(ctr.p, 0, 3 * 8, s));
  QArgs a{in.N, in.R, dgraph, ddeg, st.as<uint32_t>(), in.nstarts,
          in.start_off ? soff.as<uint32_t>() : nullptr, in.nq, in.k, in.L, 16u * in.L + 1024u,
          filt ? off.as<uint32_t>() : nullptr, filt ? lab.as<uint32_t>() : nullptr,
          filt ? qlab.as<uint32_t>() : nullptr, oi.as<uint32_t>(), od.as<float>(),
          ctr.as<unsigned long long>()};
  hipEvent_t e0, e1;
  DHIP(hipEventCreate(&e0));
  DHIP(hipEventCreate(&e1));
  DHIP(hipEventRecord(e0, s));
  const uint32_t grid = (in.nq + kWaves - 1) / kWaves;
  const size_t lds = (size_t)kWaves * kLds * 4;
  const int ps = pick_ps(in.L);
  DCHECK(with_dt_cpl(base.dtype, cpl, [&](auto dt, auto c) {
    constexpr int DT = decltype(dt)::value, CPL = decltype(c)::value;
    if (ps == 1)
      hipLaunchKernelGGL((k_query<DT, CPL, 1>), dim3(grid), dim3(kBlock), lds, s, base.rs, qr.rs, a);
    else if (ps == 2)
      hipLaunchKernelGGL((k_query<DT, CPL, 2>), dim3(grid), dim3(kBlock), lds, s, base.rs, qr.rs, a);
    else if (ps == 4)
      hipLaunchKernelGGL((k_query<DT, CPL, 4>), dim3(grid), dim3(kBlock), lds, s, base.rs, qr.rs, a);
    else if (ps == 8)
      hipLaunchKernelGGL((k_query<DT, CPL, 8>), dim3(grid), dim3(kBlock), lds, s, base.rs, qr.rs, a);
    else
      hipLaunchKernelGGL((k_query<DT, CPL, 16>), dim3(grid), dim3(kBlock), lds, s, base.rs, qr.rs, a);
    DHIP(hipGetLastError());
    return 0;
  }));
  DHIP(hipEventRecord(e1, s));
  DHIP(hipMemcpyAsync(in.ids_out, oi.p, (size_t)in.nq * in.k * 4, hipMemcpyDeviceToHost, s));
  DHIP(hipMemcpyAsync(in.d_out, od.p, (size_t)in.nq * in.k * 4, hipMemcpyDeviceToHost, s));
  unsigned long long c3[3];
  DHIP(hipMemcpyAsync(c3, ctr.p, sizeof(c3), hipMemcpyDeviceToHost, s));
  DHIP(hipStreamSynchronize(s));
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  g_qstats.kernel_ms = ms;
  g_qstats.distances = c3[0];
  g_qstats.expansions = c3[1];
  g_qstats.capped_queries = c3[2];
  return 0;
}

}  // namespace
}  // namespace dance

using namespace dance;

extern "C" {

int dance_search(const void* h_data, int dtype, uint32_t num_points, uint32_t dim, const uint32_t* h_graph,
                 const uint32_t* h_degree, uint32_t R, const uint32_t* starts, uint32_t num_starts,
                 const void* h_queries, uint32_t num_queries, uint32_t k, uint32_t L,
                 const uint32_t* point_label_offsets, const uint32_t* point_labels, const uint32_t* query_labels,
                 uint32_t* ids_out, float* dists_out) {
  return run_search(SearchIn{h_data, false, dtype, num_points, dim, h_graph, h_degree, false, R, starts, num_starts,
                             nullptr, h_queries, num_queries, k, L, point_label_offsets, point_labels, query_labels,
                             ids_out, dists_out});
}

int dance_search_resident(const void* d_data, int dtype, uint32_t num_points, uint32_t dim, const uint32_t* d_graph,
                          const uint32_t* d_degree, uint32_t R, const uint32_t* starts, uint32_t num_starts,
                          const void* h_queries, uint32_t num_queries, uint32_t k, uint32_t L,
                          const uint32_t* point_label_offsets, const uint32_t* point_labels,
                          const uint32_t* query_labels, uint32_t* ids_out, float* dists_out) {
  return run_search(SearchIn{d_data, true, dtype, num_points, dim, d_graph, d_degree, true, R, starts, num_starts,
                             nullptr, h_queries, num_queries, k, L, point_label_offsets, point_labels, query_labels,
                             ids_out, dists_out});
}

int dance_search_multistart(const void* h_data, int dtype, uint32_t num_points, uint32_t dim,
                            const uint32_t* h_graph, const uint32_t* h_degree, uint32_t R,
                            const uint32_t* start_offsets, const uint32_t* starts, const void* h_queries,
                            uint32_t num_queries, uint32_t k, uint32_t L, const uint32_t* point_label_offsets,
                            const uint32_t* point_labels, const uint32_t* query_labels, uint32_t* ids_out,
                            float* dists_out) {
  if (!start_offsets) return -1;
  return run_search(SearchIn{h_data, false, dtype, num_points, dim, h_graph, h_degree, false, R,
                             starts, num_queries ? start_offsets[num_queries] : 0u, start_offsets, h_queries,
                             num_queries, k, L, point_label_offsets, point_labels, query_labels, ids_out,
                             dists_out});
}

int dance_search_multistart_resident(const void* d_data, int dtype, uint32_t num_points, uint32_t dim,
                                     const uint32_t* d_graph, const uint32_t* d_degree, uint32_t R,
                                     const uint32_t* start_offsets, const uint32_t* starts, const void* h_queries,
                                     uint32_t num_queries, uint32_t k, uint32_t L,
                                     const uint32_t* point_label_offsets, const uint32_t* point_labels,
                                     const uint32_t* query_labels, uint32_t* ids_out, float* dists_out) {
  if (!start_offsets) return -1;
  return run_search(SearchIn{d_data, true, dtype, num_points, dim, d_graph, d_degree, true, R,
                             starts, num_queries ? start_offsets[num_queries] : 0u, start_offsets, h_queries,
                             num_queries, k, L, point_label_offsets, point_labels, query_labels, ids_out,
                             dists_out});
}

void dance_get_last_search_stats(DanceSearchStats* stats) {
  if (!stats) return;
  std::lock_guard<std::mutex> lk(g_qmu);
  *stats = g_qstats;
}

}  // extern "C"
