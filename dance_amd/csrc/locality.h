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

// Sort key of a vertex from its nearest pivots b1, b2, b3 (nearest first).
// levels = 3 orders the vertices of a cell (b1) by their second and third
// nearest pivots, i.e. by the neighbouring cells they face, so the vertices
// in flight together are closer than in vertex-id order; levels = 1 keys by
// the cell alone. Three levels need K^3 <= 2^32 (K <= 1625).
constexpr uint32_t kCellLevelsMaxK = 1625;
__host__ __device__ inline uint32_t cell_levels(uint32_t K, uint32_t levels) {
  return (levels >= 3 && K <= kCellLevelsMaxK) ? 3u : 1u;
}
__device__ __forceinline__ uint32_t cell_key(uint32_t b1, uint32_t b2, uint32_t b3, uint32_t K, uint32_t levels) {
  return levels == 3u ? (b1 * K + b2) * K + b3 : b1;
}
// Keeps the three smallest (d, k) in order, first on ties.
struct Nearest3 {
  float d1 = FLT_MAX, d2 = FLT_MAX, d3 = FLT_MAX;
  uint32_t k1 = 0, k2 = 0, k3 = 0;
  __device__ __forceinline__ void add(float d, uint32_t k) {
    if (d < d1) {
      d3 = d2;
      k3 = k2;
      d2 = d1;
      k2 = k1;
      d1 = d;
      k1 = k;
    } else if (d < d2) {
      d3 = d2;
      k3 = k2;
      d2 = d;
      k2 = k;
    } else if (d < d3) {
      d3 = d;
      k3 = k;
    }
  }
};

// Pivot k of K is row floor(k N / K) (evenly spaced).
static __global__ void k_pivots(uint32_t N, uint32_t K, uint32_t* __restrict__ piv) {
  const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < K) piv[k] = (uint32_t)(((uint64_t)k * N) / K);
}

// cell[v] = the sort key of row v's nearest pivots (first on ties; levels
// from cell_levels), vid[v] = v.
template <int DT, int CPL>
__global__ __launch_bounds__(kCellsBlock) void k_cells(RowSet rs, uint32_t N, const uint32_t* __restrict__ pivots,
                                                       uint32_t K, uint32_t levels, uint32_t* __restrict__ cell,
                                                       uint32_t* __restrict__ vid) {
  const uint32_t lane = lane_id(), grp = lane >> 3, sub = lane & 7u;
  const uint32_t w = blockIdx.x * (kCellsBlock / 64u) + wave_index();
  const uint32_t v = w * 8u + grp;
  if (w * 8u >= N) return;
  const bool act = v < N;
  uint4 xv[CPL];
  load_row<CPL>(rs, act ? v : 0u, act, sub, xv);
  Nearest3 nb;
  for (uint32_t k = 0; k < K; ++k) {
    uint4 pv[CPL];
    load_row<CPL>(rs, pivots[k], true, sub, pv);
    nb.add(octet_finish<DT, CPL>(rs, sub, xv, pv), k);
  }
  if (act && sub == 0) {
    cell[v] = cell_key(nb.k1, nb.k2, nb.k3, K, levels);
    vid[v] = v;
  }
}

}  // namespace dance
