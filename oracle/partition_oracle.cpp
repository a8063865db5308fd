// CPU oracle of the sharded build's shard assignment (dance_partition_assign;
// DiskANN's shard_data_into_clusters_only_ids and k-means assignment step,
// upstream partition.cpp, absent from the reference tree; called from
// build_merged_vamana_index, integrations/dance-diskann-78256bba.patch:1212-1260).
//
// TEST INFRASTRUCTURE ONLY: tests/ call it through oracle/oracle.py as the
// checker of the HIP kernel; product code never links it.
//
// Rule: for each point, the k_base nearest centers, nearest first, by squared
// L2 accumulated in fp64 in dimension order, acc = fma(d, d, acc) with
// d = (double)x_j - (double)c_j; strict comparisons keep the lower center
// index first on ties; a point whose distances are all NaN gets 0xFFFFFFFF.
//
// Parity status: pinned against exact integer arithmetic on integer-valued
// inputs (ties included) and against exact rational distances away from
// near-ties (tests/test_partition_oracle.py). DiskANN's own assignment (BLAS
// dot products in fp32) is absent and is not reproduced: parity unpinned
// against upstream.
#include <cmath>
#include <cstdint>
#include <vector>

extern "C" void oracle_partition_assign(const void* data, int dtype, uint64_t n, uint32_t dim, const float* centers,
                                        uint32_t K, uint32_t k_base, uint32_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)n; ++i) {
    std::vector<double> bd(k_base, INFINITY);
    std::vector<uint32_t> bi(k_base, 0xFFFFFFFFu);
    for (uint32_t k = 0; k < K; ++k) {
      double acc = 0.0;
      for (uint32_t j = 0; j < dim; ++j) {
        const double xv = dtype == 0 ? (double)static_cast<const float*>(data)[(size_t)i * dim + j]
                                     : (double)static_cast<const uint8_t*>(data)[(size_t)i * dim + j];
        const double d = xv - (double)centers[(size_t)k * dim + j];
        acc = std::fma(d, d, acc);
      }
      if (!(acc < bd[k_base - 1])) continue;
      uint32_t r = k_base - 1;
      while (r > 0 && acc < bd[r - 1]) {
        bd[r] = bd[r - 1];
        bi[r] = bi[r - 1];
        --r;
      }
      bd[r] = acc;
      bi[r] = k;
    }
    for (uint32_t r = 0; r < k_base; ++r) out[(size_t)i * k_base + r] = bi[r];
  }
}
