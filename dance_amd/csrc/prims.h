// Device primitives: exclusive scan and stable LSD radix sort of
// (key, value) pairs, hand-written for wave64. They replace the reference's
// thrust::inclusive_scan (vnew2.cu:2576-2577) and the atomic-cursor CSR fill
// (vnew2.cu:1632-1661); the sort is stable, so a list generated in source order
// comes out grouped by target with sources ascending.
#pragma once

#include "wave.h"

namespace dance {

constexpr uint32_t kScanThreads = 256;
constexpr uint32_t kScanItems = 16;
constexpr uint32_t kScanTile = kScanThreads * kScanItems;  // 4096

// Inclusive scan across the 256 threads of a block (4 waves).
__device__ __forceinline__ uint32_t block_inclusive_scan(uint32_t v, uint32_t* wsum) {
  const uint32_t lane = lane_id(), w = wave_index();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t u = (uint32_t)__shfl_up((int)v, o);
    if (lane >= (uint32_t)o) v += u;
  }
  if (lane == 63) wsum[w] = v;
  __syncthreads();
  uint32_t add = 0;
  for (uint32_t i = 0; i < w; ++i) add += wsum[i];
  __syncthreads();
  return v + add;
}

// Pass 1: per-tile exclusive scan in place; tile totals to `partial`.
static __global__ __launch_bounds__(kScanThreads) void k_scan_tile(uint32_t* __restrict__ d, size_t n,
                                                            uint32_t* __restrict__ partial) {
  __shared__ uint32_t wsum[4];
  const size_t base = (size_t)blockIdx.x * kScanTile + (size_t)threadIdx.x * kScanItems;
  uint32_t v[kScanItems];
  uint32_t s = 0;
#pragma unroll
  for (uint32_t k = 0; k < kScanItems; ++k) {
    const size_t i = base + k;
    v[k] = i < n ? d[i] : 0u;
    s += v[k];
  }
  const uint32_t incl = block_inclusive_scan(s, wsum);
  uint32_t run = incl - s;
#pragma unroll
  for (uint32_t k = 0; k < kScanItems; ++k) {
    const size_t i = base + k;
    const uint32_t x = v[k];
    if (i < n) d[i] = run;
    run += x;
  }
  if (threadIdx.x == kScanThreads - 1) partial[blockIdx.x] = incl;
}

// Pass 3: add the scanned tile offsets.
static __global__ __launch_bounds__(kScanThreads) void k_scan_add(uint32_t* __restrict__ d, size_t n,
                                                           const uint32_t* __restrict__ partial) {
  const uint32_t add = partial[blockIdx.x];
  const size_t base = (size_t)blockIdx.x * kScanTile;
  for (uint32_t k = threadIdx.x; k < kScanTile; k += kScanThreads) {
    const size_t i = base + k;
    if (i < n) d[i] += add;
  }
}

// ---------------------------------------------------------------------------
// Stable LSD radix sort, 8-bit digits. A tile is 256 threads x 16 items; each
// wave owns a contiguous 1024-item quarter of the tile and walks it in 16
// rounds of 64, so (wave, round, lane) order equals input order.
// ---------------------------------------------------------------------------
constexpr uint32_t kRadixThreads = 256;
constexpr uint32_t kRadixItems = 16;
constexpr uint32_t kRadixTile = kRadixThreads * kRadixItems;  // 4096

static __global__ __launch_bounds__(kRadixThreads) void k_radix_hist(const uint32_t* __restrict__ keys, size_t n,
                                                              uint32_t shift, uint32_t num_tiles,
                                                              uint32_t* __restrict__ hist) {
  __shared__ uint32_t h[256];
  h[threadIdx.x] = 0u;
  __syncthreads();
  const size_t base = (size_t)blockIdx.x * kRadixTile;
  for (uint32_t k = threadIdx.x; k < kRadixTile; k += kRadixThreads) {
    const size_t i = base + k;
    if (i < n) atomicAdd(&h[(keys[i] >> shift) & 255u], 1u);
  }
  __syncthreads();
  hist[(size_t)threadIdx.x * num_tiles + blockIdx.x] = h[threadIdx.x];
}

// Scatter of one pass: items get the same output positions as a direct
// scatter (digit base of the tile + rank among the tile's items of that digit,
// in input order), but the tile is first reordered by digit in LDS so that
// consecutive threads write consecutive addresses of a digit's run.
static __global__ __launch_bounds__(kRadixThreads) void k_radix_scatter(const uint32_t* __restrict__ keys,
                                                                 const uint32_t* __restrict__ vals, size_t n,
                                                                 uint32_t shift, uint32_t num_tiles,
                                                                 const uint32_t* __restrict__ hist_scanned,
                                                                 uint32_t* __restrict__ okeys,
                                                                 uint32_t* __restrict__ ovals) {
  __shared__ uint32_t wcnt[4][256];
  __shared__ uint32_t gbase[256];
  __shared__ uint32_t toff[256];
  __shared__ uint32_t wsum[4];
  __shared__ uint32_t skey[kRadixTile];
  __shared__ uint32_t sval[kRadixTile];
  const uint32_t lane = lane_id(), w = wave_index();
  for (uint32_t i = threadIdx.x; i < 4 * 256; i += kRadixThreads) (&wcnt[0][0])[i] = 0u;
  gbase[threadIdx.x] = hist_scanned[(size_t)threadIdx.x * num_tiles + blockIdx.x];
  __syncthreads();
  const size_t tile0 = (size_t)blockIdx.x * kRadixTile;
  const size_t base = tile0 + (size_t)w * (64 * kRadixItems);
  uint32_t kk[kRadixItems], vv[kRadixItems], rk[kRadixItems];
  const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
  for (uint32_t r = 0; r < kRadixItems; ++r) {
    const size_t i = base + (size_t)r * 64 + lane;
    const bool in = i < n;
    const uint32_t key = in ? keys[i] : 0xFFFFFFFFu;
    kk[r] = key;
    vv[r] = in ? vals[i] : 0u;
    const uint32_t dig = (key >> shift) & 255u;
    uint64_t peers = wballot(in);
#pragma unroll
    for (uint32_t b = 0; b < 8; ++b) {
      const uint64_t m = wballot(((dig >> b) & 1u) != 0u);
      peers &= ((dig >> b) & 1u) ? m : ~m;
    }
    const uint32_t before = (uint32_t)__popcll((unsigned long long)(peers & lt));
    const uint32_t prior = in ? wcnt[w][dig] : 0u;
    wave_sync();
    // The highest peer publishes the new running count for this digit.
    if (in && (peers >> lane) == 1ull) wcnt[w][dig] = prior + before + 1u;
    wave_sync();
    rk[r] = prior + before;
  }
  __syncthreads();
  {
    const uint32_t dgt = threadIdx.x;
    uint32_t run = 0;
    for (uint32_t q = 0; q < 4; ++q) {
      const uint32_t c = wcnt[q][dgt];
      wcnt[q][dgt] = run;
      run += c;
    }
    // offset of this digit's run inside the tile
    toff[dgt] = block_inclusive_scan(run, wsum) - run;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t r = 0; r < kRadixItems; ++r) {
    const size_t i = base + (size_t)r * 64 + lane;
    if (i < n) {
      const uint32_t dig = (kk[r] >> shift) & 255u;
      const uint32_t li = toff[dig] + wcnt[w][dig] + rk[r];
      skey[li] = kk[r];
      sval[li] = vv[r];
    }
  }
  __syncthreads();
  const uint32_t cnt = (uint32_t)min((size_t)kRadixTile, n - tile0);
  for (uint32_t i = threadIdx.x; i < cnt; i += kRadixThreads) {
    const uint32_t key = skey[i];
    const uint32_t dig = (key >> shift) & 255u;
    const size_t pos = (size_t)gbase[dig] + (i - toff[dig]);
    okeys[pos] = key;
    ovals[pos] = sval[i];
  }
}

}  // namespace dance
