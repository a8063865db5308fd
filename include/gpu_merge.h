/* Shard-graph merge, implemented by libdance_hip.so for gfx950.
 *
 * Drop-in for /root/reference/include/gpu_merge.h:8-12 (implementation
 * reference: src/gpu_merge.cu:351-790): same namespace, name, argument order
 * and meaning, output files and return codes.
 *
 * Inputs: nshards DiskANN in-memory graphs "<vamana_prefix><i><vamana_suffix>"
 * (header: u64 file size, u32 width, u32 medoid, u64 frozen points, which must
 * be 0; then per local node a u32 degree and that many u32 local neighbour ids)
 * and their id maps "<idmaps_prefix><i><idmaps_suffix>" (u32 count, u32 1,
 * then count u32 global ids, local index -> global id).
 *
 * Output graph (output_vamana): one row per global id 0 .. max_id, each row the
 * union of its mapped shard edges without self loops or duplicates, ranked by
 * a 32-bit mix of (source, target, seed) (ties: smaller target id) and cut to
 * max_degree; header width = max_degree, medoid = the last shard's medoid as a
 * global id, frozen = 0. medoids_file: u32 nshards, u32 1, then each shard's
 * medoid as a global id. DISKANN_GPU_MERGE_HASH_SEED overrides the rank seed
 * (default 0x9e3779b97f4a7c15); DISKANN_GPU_MERGE_BUCKETS and
 * DISKANN_GPU_MERGE_BUCKET_EDGES split the source range into buckets (the
 * output does not depend on them).
 *
 * Returns 0 on success; -2 unreadable id map, -3 bad or missing graph header
 * or frozen points, -4 shard medoid out of range, -6 truncated graph body,
 * -7 a local neighbour id outside its shard, -10/-11 medoid / output file not
 * writable, -1 any other parameter or HIP runtime error (message on stderr).
 * Synchronous; uses the caller's current HIP device. */
#ifndef DANCE_GPU_MERGE_H
#define DANCE_GPU_MERGE_H

#include <cstdint>
#include <string>

namespace diskann
{

int merge_shards_gpu(const std::string &vamana_prefix, const std::string &vamana_suffix,
                     const std::string &idmaps_prefix, const std::string &idmaps_suffix, uint64_t nshards,
                     uint32_t max_degree, const std::string &output_vamana, const std::string &medoids_file);

}

#endif
