// Shard assignment for the sharded build: every point's k_base nearest of K
// centers (DiskANN's shard_data_into_clusters_only_ids and the assignment
// step of its k-means, upstream partition.cpp / math_utils.cpp, called from
// build_merged_vamana_index, /root/reference/integrations/dance-diskann-78256bba.patch:1212-1260).
//
// Distance: squared L2 in fp64, acc = fma(d, d, acc) over the dimensions in
// order with d = (double)x_j - (double)c_j; ties go to the lower center index.
// Every fp32 / u8 value is exact in fp64 and the order is fixed, so the
// result does not depend on the launch shape. A point whose distances are
// all NaN gets DANCE_INV.
//
// Layout: one wave per 64 points; the wave stages its 64 rows in LDS as fp32
// (row stride dim + 1 words, so the 64 lanes reading element j of their own
// rows hit distinct banks), then each lane walks the centers, which every
// lane reads at the same address (scalar loads).

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "../../include/dance_hip.h"
#include "host_common.h"

namespace dance {
namespace {

constexpr uint32_t kAssignPoints = 64;   // points per workgroup (one wave)
constexpr uint32_t kAssignMaxDim = 255;  // 64 x (dim + 1) fp32 words fit 64 KB of LDS
constexpr uint32_t kAssignMaxK = 8;      // nearest centers kept per point
constexpr uint64_t kAssignChunk = 1ull << 22;  // points per upload

template <int DT>
__global__ __launch_bounds__(kAssignPoints) void k_assign(const uint8_t* __restrict__ rows, uint32_t n, uint32_t dim,
                                                          const float* __restrict__ centers, uint32_t K,
                                                          uint32_t k_base, uint32_t* __restrict__ out) {
  extern __shared__ float xs[];
  const uint32_t lane = threadIdx.x;
  const uint32_t p0 = blockIdx.x * kAssignPoints;
  const uint32_t np = min(kAssignPoints, n - p0);
  const uint32_t stride = dim + 1u;
  for (uint32_t p = 0; p < np; ++p) {
    const size_t r = (size_t)(p0 + p) * dim;
    for (uint32_t j = lane; j < dim; j += kAssignPoints) {
      float v;
      if constexpr (DT == DANCE_F32)
        v = reinterpret_cast<const float*>(rows)[r + j];
      else
        v = (float)rows[r + j];
      xs[p * stride + j] = v;
    }
  }
  __syncthreads();
  if (lane >= np) return;
  const float* x = xs + lane * stride;
  double bd[kAssignMaxK];
  uint32_t bi[kAssignMaxK];
#pragma unroll
  for (uint32_t r = 0; r < kAssignMaxK; ++r) {
    bd[r] = __builtin_inf();
    bi[r] = DANCE_INV;
  }
  for (uint32_t k = 0; k < K; ++k) {
    const float* c = centers + (size_t)k * dim;
    double acc = 0.0;
    for (uint32_t j = 0; j < dim; ++j) {
      const double d = (double)x[j] - (double)c[j];
      acc = __builtin_fma(d, d, acc);
    }
    // insertion into the ascending k_base best (unrolled, so the arrays stay
    // in registers); strict < keeps the lower center index first on ties
    if (acc < bd[k_base - 1]) {
      uint32_t pos = k_base - 1;
#pragma unroll
      for (int r = (int)kAssignMaxK - 1; r > 0; --r) {
        if ((uint32_t)r == pos && acc < bd[r - 1]) {
          bd[r] = bd[r - 1];
          bi[r] = bi[r - 1];
          pos = (uint32_t)r - 1;
        }
      }
#pragma unroll
      for (uint32_t r = 0; r < kAssignMaxK; ++r)
        if (r == pos) {
          bd[r] = acc;
          bi[r] = k;
        }
    }
  }
  const size_t o = (size_t)(p0 + lane) * k_base;
#pragma unroll
  for (uint32_t r = 0; r < kAssignMaxK; ++r)
    if (r < k_base) out[o + r] = bi[r];
}

}  // namespace
}  // namespace dance

extern "C" int dance_partition_assign(const void* h_data, int dtype, uint64_t num_points, uint32_t dim,
                                      const float* h_centers, uint32_t num_centers, uint32_t k_base,
                                      uint32_t* h_assign) {
  using namespace dance;
  if (!h_data || !h_centers || !h_assign || dim == 0 || num_centers == 0 || k_base == 0 ||
      k_base > kAssignMaxK || k_base > num_centers || (dtype != DANCE_F32 && dtype != DANCE_U8)) {
    std::fprintf(stderr, "[dance_partition_assign] invalid arguments (dim=%u centers=%u k_base=%u dtype=%d)\n", dim,
                 num_centers, k_base, dtype);
    return -1;
  }
  if (dim > kAssignMaxDim) {
    std::fprintf(stderr, "[dance_partition_assign] dim=%u exceeds %u\n", dim, kAssignMaxDim);
    return -1;
  }
  if (num_points == 0) return 0;
  const uint32_t eb = dtype == DANCE_F32 ? 4u : 1u;
  const uint64_t chunk = std::min<uint64_t>(num_points, kAssignChunk);
  hipStream_t s = nullptr;
  DHIP(hipStreamCreate(&s));
  struct Guard {
    hipStream_t s;
    ~Guard() { (void)hipStreamDestroy(s); }
  } guard{s};
  DevBuf rows, cen, out;
  DCHECK(rows.alloc((size_t)chunk * dim * eb));
  DCHECK(cen.alloc((size_t)num_centers * dim * 4));
  DCHECK(out.alloc((size_t)chunk * k_base * 4));
  DHIP(hipMemcpyAsync(cen.p, h_centers, (size_t)num_centers * dim * 4, hipMemcpyHostToDevice, s));
  const size_t lds = (size_t)kAssignPoints * (dim + 1) * 4;
  for (uint64_t b = 0; b < num_points; b += chunk) {
    const uint32_t n = (uint32_t)std::min<uint64_t>(chunk, num_points - b);
    DHIP(hipMemcpyAsync(rows.p, static_cast<const uint8_t*>(h_data) + (size_t)b * dim * eb, (size_t)n * dim * eb,
                        hipMemcpyHostToDevice, s));
    const uint32_t grid = (n + kAssignPoints - 1) / kAssignPoints;
    if (dtype == DANCE_F32)
      hipLaunchKernelGGL(k_assign<DANCE_F32>, dim3(grid), dim3(kAssignPoints), lds, s, rows.as<const uint8_t>(), n,
                         dim, cen.as<const float>(), num_centers, k_base, out.as<uint32_t>());
    else
      hipLaunchKernelGGL(k_assign<DANCE_U8>, dim3(grid), dim3(kAssignPoints), lds, s, rows.as<const uint8_t>(), n,
                         dim, cen.as<const float>(), num_centers, k_base, out.as<uint32_t>());
    DHIP(hipGetLastError());
    DHIP(hipMemcpyAsync(h_assign + (size_t)b * k_base, out.p, (size_t)n * k_base * 4, hipMemcpyDeviceToHost, s));
  }
  DHIP(hipStreamSynchronize(s));
  return 0;
}
