// Device kernels of the stitched build (per-label standard builds stitched
// into one global graph; reference apps/utils/gpu_stitched_vamana_index.cpp,
// whose label loop gathers rows, builds, and remaps on the host, :276-341).
// Here the rows of a label are gathered and the local graph is remapped to
// global ids on the device; the global graph never leaves HBM until the end.
#pragma once

#include "wave.h"

namespace dance {

// Rows ids[0..m) of the packed N x dim input (elements of SrcT) into the
// padded row layout of the build (stride16 chunks of 16 bytes per row, zero
// padding; DstT = _Float16 converts with round to nearest even, as the
// FAST_SMALL upload does). One thread per destination element.
template <typename SrcT, typename DstT>
__global__ void k_gather_rows(const SrcT* __restrict__ src, uint32_t dim, const uint32_t* __restrict__ ids, uint32_t m,
                              DstT* __restrict__ dst, uint32_t dst_elems_per_row) {
  const uint64_t t = (uint64_t)grid_block() * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)m * dst_elems_per_row) return;
  const uint32_t r = (uint32_t)(t / dst_elems_per_row), e = (uint32_t)(t % dst_elems_per_row);
  DstT v = (DstT)0;
  if (e < dim) v = (DstT)src[(size_t)ids[r] * dim + e];
  dst[t] = v;
}

__global__ void k_fill_u32(uint32_t* __restrict__ p, uint64_t n, uint32_t v) {
  const uint64_t t = (uint64_t)grid_block() * blockDim.x + threadIdx.x;
  if (t < n) p[t] = v;
}

struct RemapArgs {
  const uint32_t* local;      // m x Rs local graph (local ids, INVALID-padded)
  const uint32_t* local_deg;  // m
  const uint32_t* ids;        // m: local id -> global id
  uint32_t m, Rs;
  uint32_t take;              // at most `take` leading entries of each local row (Rstitched)
  uint32_t* graph;            // N x row_cap global rows
  uint32_t* degree;           // N
  uint32_t row_cap;
  unsigned long long* ctr;    // [0] invalid local ids, [1] self loops, [2] repeated ids
};

// One wave per local point i, appending to global row ids[i] in local-row
// order: entry j is dropped when it is not a valid local id, when it maps to
// the row's own point, or when the global row already holds its global id
// (from an earlier label or an earlier entry of this row); kept entries go
// after the row's current end. Entries are taken 64 at a time, each lane
// testing its entry against the row (in LDS) and the earlier lanes' ids.
// The host sizes row_cap for every label of a point, so appends never
// overflow it.
constexpr uint32_t kRemapWaves = 4;
__global__ __launch_bounds__(64 * kRemapWaves) void k_stitch_remap(RemapArgs a) {
  __shared__ uint32_t s_row[kRemapWaves][256];
  __shared__ uint32_t s_new[kRemapWaves][64];
  const uint32_t w = wave_index(), lane = lane_id();
  const uint32_t i = grid_block() * kRemapWaves + w;
  if (i >= a.m) return;
  const uint32_t me = a.ids[i];
  const uint32_t deg = min(min(a.local_deg[i], a.take), a.Rs);
  uint32_t* row = a.graph + (size_t)me * a.row_cap;
  uint32_t have = uni_u(a.degree[me]);
  uint32_t n_inv = 0, n_self = 0, n_dup = 0;
  for (uint32_t b = 0; b < deg; b += 64) {
    // current row content into LDS (row_cap <= 256 is checked on the host)
    for (uint32_t k = lane; k < have; k += 64) s_row[w][k] = row[k];
    const uint32_t j = b + lane;
    const bool in = j < deg;
    const uint32_t nb = in ? a.local[(size_t)i * a.Rs + j] : DANCE_INV;
    const bool valid = in && nb < a.m;
    const uint32_t g = valid ? a.ids[nb] : DANCE_INV;
    const bool self = valid && g == me;
    const bool cand = valid && !self;
    s_new[w][lane] = cand ? g : DANCE_INV;
    wave_sync();
    bool dup = false;
    if (cand) {
      for (uint32_t k = 0; k < have && !dup; ++k) dup = s_row[w][k] == g;
      for (uint32_t k = 0; k < lane && !dup; ++k) dup = s_new[w][k] == g;
    }
    const bool keep = cand && !dup;
    const uint64_t km = wballot(keep);
    if (keep) row[have + mbcnt64(km)] = g;
    have += popc64(km);
    n_inv += popc64(wballot(in && !valid));
    n_self += popc64(wballot(self));
    n_dup += popc64(wballot(cand && dup));
    wave_sync();
  }
  if (lane == 0) {
    a.degree[me] = have;
    if (n_inv) atomicAdd(&a.ctr[0], (unsigned long long)n_inv);
    if (n_self) atomicAdd(&a.ctr[1], (unsigned long long)n_self);
    if (n_dup) atomicAdd(&a.ctr[2], (unsigned long long)n_dup);
  }
}

}  // namespace dance
