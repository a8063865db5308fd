/* Standard GPU Vamana builder ABI, implemented by libdance_hip.so for gfx950.
 *
 * Drop-in for /root/reference/include/gpu_vamana_builder.h: same symbol
 * names, argument order and meaning, struct layout and return codes (0 on
 * success, -1 on invalid parameters or a runtime error, message on stderr).
 * The field order of GPUVamanaStats is load-bearing: callers copy it by value
 * (reference: include/gpu_vamana_builder.h:11-28). Layout is checked by
 * static_assert in dance_amd/csrc/vnew2_build.hip.
 *
 * Caller owns h_graph (num_points * R uint32, rows padded with 0xFFFFFFFF
 * after the degree) and h_degree (num_points). Inputs are read-only. Builds
 * are synchronous, use the caller's current HIP device, and are not
 * thread-safe: the "last medoid / last stats" getters read process globals,
 * as in the reference (src/gpu_vamana_vnew2.cu:2149-2168). */
#ifndef DANCE_GPU_VAMANA_BUILDER_H
#define DANCE_GPU_VAMANA_BUILDER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct GPUVamanaStats {
    double medoid_seconds;
    double h2d_seconds;
    double search_online_insert_seconds;
    double reverse_seconds;
    double final_prune_seconds;
    double d2h_seconds;
    double gpu_build_seconds;
    uint64_t distance_computations;
    uint64_t online_insert_attempts;
    uint64_t online_insert_mutations;
    uint64_t reverse_candidate_overflows;
    uint64_t reverse_proposals;
    uint64_t reverse_touched_rows;
    double reverse_csr_seconds;
    uint32_t selective_active_nodes;
} GPUVamanaStats;

/* "v8" build (reference: include/gpu_vamana_builder.h:30-48,
 * src/gpu_vamana_uint8.cu:2437-3120), the sharded pipeline's default shard
 * builder. Same schedule, search, online insert, reverse merge and prune as
 * vnew2, without the reverse heavy cap in any profile; the float entry stores
 * fp16 rows under the fp16 profiles, as vnew2 does. */
int gpu_vamana_build(const uint8_t *h_data, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t L,
                     uint32_t C, uint32_t STEPS, uint32_t *h_graph, uint32_t *h_degree);
int gpu_vamana_build_float(const float *h_data, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t L,
                           uint32_t C, uint32_t STEPS, uint32_t *h_graph, uint32_t *h_degree);

/* vnew2 standard build (reference: include/gpu_vamana_builder.h:50-68,
 * src/gpu_vamana_vnew2.cu:2857-2917). The float entry stores fp32 rows under
 * the QUALITY profile and fp16 rows under FAST_SMALL (dance_set_profile). */
int gpu_vamana_vnew2_build(const uint8_t *h_data, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t L,
                           uint32_t C, uint32_t STEPS, uint32_t *h_graph, uint32_t *h_degree);
int gpu_vamana_vnew2_build_float(const float *h_data, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t L,
                                 uint32_t C, uint32_t STEPS, uint32_t *h_graph, uint32_t *h_degree);

/* Device hand-off variants (reference: include/gpu_vamana_builder.h:70-75,
 * src/gpu_vamana_vnew2_handoff.cu:110-151): the build keeps the uploaded
 * vectors (num_points x dim), the graph (num_points x R) and the degrees in
 * device memory and transfers ownership to the caller, who releases each
 * with hipFree. */
int gpu_vamana_vnew2_build_device(const uint8_t *h_data, uint32_t num_points, uint32_t dim, uint32_t R,
                                  uint32_t L, uint32_t C, uint32_t STEPS, uint8_t **d_data, uint32_t **d_graph,
                                  uint32_t **d_degree);
int gpu_vamana_vnew2_build_device_float(const float *h_data, uint32_t num_points, uint32_t dim, uint32_t R,
                                        uint32_t L, uint32_t C, uint32_t STEPS, float **d_data,
                                        uint32_t **d_graph, uint32_t **d_degree);

/* Last-build getters (reference: include/gpu_vamana_builder.h:78-81). The
 * gpu_vamana_* pair reports the last v8 build, the gpu_vamana_vnew2_* pair the
 * last vnew2 build (hand-off and resident builds included). */
uint32_t gpu_vamana_get_last_medoid(void);
void gpu_vamana_get_last_stats(GPUVamanaStats *stats);
uint32_t gpu_vamana_vnew2_get_last_medoid(void);
void gpu_vamana_vnew2_get_last_stats(GPUVamanaStats *stats);

#ifdef __cplusplus
}
#endif

#endif
