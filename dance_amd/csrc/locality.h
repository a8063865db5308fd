// Locality schedule shared by the standard and the filtered builds: each
// vertex's nearest of K pivot rows (one octet per vertex, eight vertices per
// wave). Vertices sorted by cell make the waves in flight work on
// neighbouring vertices, whose searches, candidate rows and reverse sources
// overlap in L2 and the MALL. The schedule only changes the order in which
// independent vertices are processed, never a result.
#pragma once

#include "wave.h"

namespace dance {

constexpr uint32_t kCellsBlock = 256;  // 4 waves, 32 vertices per workgroup

inline uint32_t cells_grid(uint32_t N) { return (N + 31u) / 32u; }

// Pivot k of K is row floor(k N / K) (evenly spaced).
static __global__ void k_pivots(uint32_t N, uint32_t K, uint32_t* __restrict__ piv) {
  const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < K) piv[k] = (uint32_t)(((uint64_t)k * N) / K);
}

// cell[v] = the nearest pivot of row v (first on ties), vid[v] = v.
template <int DT, int CPL>
__global__ __launch_bounds__(kCellsBlock) void k_cells(RowSet rs, uint32_t N, const uint32_t* __restrict__ pivots,
                                                       uint32_t K, uint32_t* __restrict__ cell,
                                                       uint32_t* __restrict__ vid) {
  const uint32_t lane = lane_id(), grp = lane >> 3, sub = lane & 7u;
  const uint32_t w = blockIdx.x * (kCellsBlock / 64u) + wave_index();
  const uint32_t v = w * 8u + grp;
  if (w * 8u >= N) return;
  const bool act = v < N;
  uint4 xv[CPL];
  load_row<CPL>(rs, act ? v : 0u, act, sub, xv);
  float best = FLT_MAX;
  uint32_t bi = 0;
  for (uint32_t k = 0; k < K; ++k) {
    uint4 pv[CPL];
    load_row<CPL>(rs, pivots[k], true, sub, pv);
    const float d = octet_finish<DT, CPL>(rs, sub, xv, pv);
    if (d < best) {
      best = d;
      bi = k;
    }
  }
  if (act && sub == 0) {
    cell[v] = bi;
    vid[v] = v;
  }
}

}  // namespace dance
