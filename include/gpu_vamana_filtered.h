/* Label-filtered GPU Vamana builder ABI, implemented by libdance_hip.so for
 * gfx950.
 *
 * Drop-in for /root/reference/include/gpu_vamana_filtered.h: same symbol
 * names, argument order and meaning, struct layout and return codes. The
 * build is the reference's release path ("canonical_v2",
 * src/gpu_vamana_filtered.cu:6511-7067 and :5663-6483): a deterministic
 * random backbone (degree min(16, R), seed 42), then three rounds of
 * per-label exact-label searches, a union-label search, candidate merge with
 * a per-label quota, FilteredRobustPrune, and an exact reverse-CSR repair.
 * Float vectors are searched as fp16 (round to nearest even), uint8 vectors
 * as integers.
 *
 * Labels: point p carries point_labels[point_label_offsets[p] ..
 * point_label_offsets[p+1]), sorted ascending without repeats;
 * point_label_offsets has num_points+1 entries with
 * point_label_offsets[num_points] == total_label_count. label_to_start_id
 * has max(1, num_labels) entries (0xFFFFFFFF or >= num_points: no entry
 * point). universal_label_id matches every label in the diagnostics and is
 * never searched as a task. query_anchor_* are accepted and unused, as in
 * the reference's release path.
 *
 * Returns 0 on success; -1 on null pointers, invalid sizes (num_points, dim,
 * R or L zero, C < R), malformed label offsets, labels of a point that are
 * not strictly ascending, or a runtime error; 1 when the
 * GPU work capacity min(C, 128) per point cannot hold the exact reverse CSR
 * (min(C, 128) < 2 * R), as the reference does. Messages go to stderr.
 * Caller owns h_graph (num_points * PR, rows padded with 0xFFFFFFFF) and
 * h_degree (num_points). PR is R, or min(R, v) when the environment variable
 * DISKANN_GPU_FILTERED_PUBLISH_DEGREE holds v > 0 (atoi): below R the built
 * graph is shortlisted and pruned to PR per row, then rows with reverse
 * edges are rebuilt from their row plus those sources and pruned again (the
 * publish step, reference gpu_vamana_filtered.cu:6328-6432). Builds are synchronous and serialized; the last
 * stats are a process global, as in the reference. */
#ifndef DANCE_GPU_VAMANA_FILTERED_H
#define DANCE_GPU_VAMANA_FILTERED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Field order and types are load-bearing (callers copy the struct by value):
 * reference include/gpu_vamana_filtered.h:11-77. Fields of reference stages
 * that the release path does not run stay 0. */
typedef struct GPUFilteredVamanaStats {
    double gpu_build_seconds;
    double label_h2d_seconds;
    double graph_build_seconds;
    double diagnostics_seconds;
    double d2h_seconds;
    double peak_gpu_mem_gb;
    double backbone_seconds;
    double task_generation_seconds;
    double filtered_search_seconds;
    double ordinary_search_seconds;
    double merge_seconds;
    double forward_prune_seconds;
    double csr_reverse_seconds;
    double reverse_prune_seconds;
    double compaction_seconds;

    uint64_t filtered_search_distance_count;
    uint64_t unfiltered_search_distance_count;
    uint64_t label_check_count;
    uint64_t label_reject_count;
    uint64_t filtered_candidate_count;
    uint64_t unfiltered_candidate_count;
    uint64_t merged_candidate_count;
    uint64_t active_rows;
    uint64_t original_neighbor_count;
    uint64_t filtered_seed_count;
    uint64_t filtered_visited_count;
    uint64_t filtered_visited_reserved_count;
    uint64_t filtered_top_reserved_count;
    uint64_t bridge_reserved_count;
    uint64_t unfiltered_reserved_count;
    uint64_t filtered_reserved_count;
    uint64_t label_occlusion_blocked_count;
    uint64_t geometry_occluded_count;
    uint64_t candidate_rejected_by_label_count;
    uint64_t refill_count;
    uint64_t filtered_prune_reject_count;
    uint64_t universal_label_pass_count;
    uint64_t final_prune_rows;
    uint64_t reverse_edges;
    uint64_t reverse_touched_rows;
    uint64_t filtered_reverse_edges;
    uint64_t filtered_reverse_touched_rows;
    uint64_t filtered_reverse_candidates_kept;
    uint64_t filtered_reverse_pruned_rows;

    double avg_common_label_out_degree;
    double common_label_degree_before_avg;
    double common_label_degree_after_avg;
    double active_rows_frac;
    uint32_t low_common_label_degree_count;
    uint32_t low_common_before;
    uint32_t low_common_after;
    uint32_t out_degree_min;
    uint32_t out_degree_max;
    double out_degree_avg;
    uint32_t common_label_degree_min;
    uint32_t common_label_degree_max;
    uint32_t invalid_neighbor_count;
    uint32_t self_loop_count;
    double prune_output_degree_avg;
    uint32_t filtered_seed_source;
    uint32_t semantic_stage;
    uint32_t semantic_complete;
} GPUFilteredVamanaStats;

/* Reference: include/gpu_vamana_filtered.h:79-99, src/gpu_vamana_filtered.cu:8793-8820. */
int gpu_vamana_filtered_build_uint8(const uint8_t *h_data, uint32_t num_points, uint32_t dim, uint32_t R,
                                    uint32_t L, uint32_t filtered_L, uint32_t C, uint32_t STEPS, float alpha,
                                    const uint32_t *point_label_offsets, const uint32_t *point_labels,
                                    uint32_t total_label_count, const uint32_t *label_to_start_id,
                                    uint32_t num_labels, uint32_t universal_label_id, uint32_t global_start_id,
                                    const uint32_t *query_anchor_offsets, const uint32_t *query_anchor_ids,
                                    uint32_t query_anchor_count, uint32_t *h_graph, uint32_t *h_degree);

/* Reference: include/gpu_vamana_filtered.h:101-121, src/gpu_vamana_filtered.cu:8822-8849. */
int gpu_vamana_filtered_build_float(const float *h_data, uint32_t num_points, uint32_t dim, uint32_t R,
                                    uint32_t L, uint32_t filtered_L, uint32_t C, uint32_t STEPS, float alpha,
                                    const uint32_t *point_label_offsets, const uint32_t *point_labels,
                                    uint32_t total_label_count, const uint32_t *label_to_start_id,
                                    uint32_t num_labels, uint32_t universal_label_id, uint32_t global_start_id,
                                    const uint32_t *query_anchor_offsets, const uint32_t *query_anchor_ids,
                                    uint32_t query_anchor_count, uint32_t *h_graph, uint32_t *h_degree);

/* Reference: include/gpu_vamana_filtered.h:123, src/gpu_vamana_filtered.cu:8851-8855. */
void gpu_vamana_filtered_get_last_stats(GPUFilteredVamanaStats *stats);

#ifdef __cplusplus
}
#endif

#endif
