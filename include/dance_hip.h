/* Extension entry points of libdance_hip.so beyond the reference's public
 * headers. The reference ABI itself (gpu_vamana_builder.h,
 * gpu_vamana_filtered.h) is declared unchanged in the sibling headers; these
 * entry points serve the bench (device-resident inputs), per-kernel
 * measurement, and stage-level parity tests. Each stage hook runs exactly the
 * kernel the production build uses, on host buffers, and cites the reference
 * kernel it replaces. All return 0 on success and -1 on error (message on
 * stderr), like the reference ABI. */
#ifndef DANCE_HIP_H
#define DANCE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of the vector rows. */
enum { DANCE_DTYPE_F32 = 0, DANCE_DTYPE_U8 = 1, DANCE_DTYPE_F16 = 2 };

/* Most build iterations the library runs (the reference's VAMANA_ITERS,
 * include/gpu_vamana_config.h:78-79, compile-time there; here the run-time
 * setting DANCE_VAMANA_ITERS, 1..DANCE_MAX_ITERS, default 4), and the length
 * of the per-iteration arrays below. */
#define DANCE_MAX_ITERS 8

/* Per-kernel timings (HIP events on the build stream) and algorithmic work
 * counted on the device by each wave. Bytes are algorithmic: one vector row
 * per distance gathered, plus adjacency and work rows as documented in
 * dance_amd/csrc/vnew2_build.hip. init_ms covers the quantization and the
 * locality schedule, and the random initial graph's kernel at L > 128 (at
 * L <= 128 the first search launch computes that graph itself). */
typedef struct DanceKernelProfile {
    double medoid_ms, init_ms, search_ms, reverse_ms, merge_ms, prune_ms, total_ms;
    uint32_t iterations;
    uint32_t vector_bytes;
    uint64_t search_dist, insert_dist, expansions, vis_skips;
    uint64_t merge_dist, prune_dist, reverse_edges, touched_rows;
    double search_bytes, merge_bytes, prune_bytes, reverse_bytes;
    /* Search-kernel phase cycles (zero unless built with DANCE_SEARCH_TIMING=1). */
    uint64_t cyc_select, cyc_insert, cyc_dist, cyc_pool, cyc_seed, cyc_total;
    /* Quantized lower bound of the search (fp32/fp16 rows of <= 112 dims):
     * candidates tested, and those whose exact distance it made unnecessary
     * (proved >= the pool threshold). DANCE_QBOUND=0 disables the bound;
     * DANCE_QBOUND_ITERS selects the iterations (bit i = iteration i);
     * unset, the first iteration and, when the iteration before it computed
     * more than 24 candidate distances per expansion, the last. */
    uint64_t bound_checks, bound_skips;
    /* The same bound in RobustPrune: pairs tested, and pairs it proved far
     * enough that the candidate survives (DANCE_QBOUND_PRUNE_ITERS selects
     * the iterations). */
    uint64_t prune_bound_checks, prune_bound_skips;
    /* per iteration (launch order; entries from `iterations` on are 0):
     * search and prune launch times in ms */
    double search_iter_ms[DANCE_MAX_ITERS], prune_iter_ms[DANCE_MAX_ITERS];
    /* per iteration: the counters above split by launch, and the algorithmic
     * bytes of each search and prune launch (the totals above are their sums) */
    uint64_t search_dist_iter[DANCE_MAX_ITERS], insert_dist_iter[DANCE_MAX_ITERS],
        expansions_iter[DANCE_MAX_ITERS], bound_checks_iter[DANCE_MAX_ITERS], bound_skips_iter[DANCE_MAX_ITERS];
    uint64_t merge_dist_iter[DANCE_MAX_ITERS], prune_dist_iter[DANCE_MAX_ITERS],
        prune_bound_checks_iter[DANCE_MAX_ITERS], prune_bound_skips_iter[DANCE_MAX_ITERS];
    double search_bytes_iter[DANCE_MAX_ITERS], prune_bytes_iter[DANCE_MAX_ITERS];
    /* RobustPrune selection rounds (vertices x rounds) and the rounds that
     * computed at least one exact pair distance, over all iterations; phase
     * cycles of the rank-mask prune (zero unless built with
     * DANCE_SEARCH_TIMING=1): ranking, bound tiles, selection rounds, fill and
     * write-back, summed over waves */
    uint64_t prune_rounds, prune_exact_rounds;
    uint64_t cyc_prune_rank, cyc_prune_gram, cyc_prune_rounds, cyc_prune_fill;
    /* The insert bound (fp32/fp16 rows of <= 112 dims, C <= 128, L <= 128):
     * online-insert occlusion pairs tested on the code rows, and those whose
     * exact distance the code-row bounds made unnecessary, in total and per
     * iteration. DANCE_INSERT_BOUND_ITERS selects the iterations (bit i =
     * iteration i, among those with the search bound on; default 0x1). */
    uint64_t insert_bound_checks, insert_bound_skips;
    uint64_t insert_bound_checks_iter[DANCE_MAX_ITERS], insert_bound_skips_iter[DANCE_MAX_ITERS];
} DanceKernelProfile;

/* Full standard (vnew2) build with the vectors already resident in device
 * memory (row-major N x dim of `dtype`) and device outputs d_graph (N x R,
 * 0xFFFFFFFF-padded rows) and d_degree (N). Same algorithm, parameters and
 * errors as gpu_vamana_vnew2_build (reference: src/gpu_vamana_vnew2.cu:2170-2855);
 * used by the bench so the timed region excludes PCIe. */
int dance_vamana_build_resident(const void *d_data, int dtype, uint32_t num_points, uint32_t dim, uint32_t R,
                                uint32_t L, uint32_t C, uint32_t STEPS, uint32_t *d_graph, uint32_t *d_degree);

/* dance_vamana_build_resident without any device allocation. No counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (tight serving loops, harnesses that forbid hipMalloc). It cannot be
 * recorded into a HIP graph: the build waits on its stream and reads the
 * medoid scores and the locality order back mid-build. Every buffer the
 * build needs beyond the caller's inputs and outputs comes from a per-GPU
 * scratch array of 256 MiB that the library holds until the process ends
 * (at R=64, C=80, fp32 rows of 96 dimensions that is about 120k vertices);
 * every process that loads the library reserves it on each GPU it uses.
 * Larger inputs return -1 with a message. The
 * work runs on the null stream and creates no event, so the stage times of
 * dance_get_last_kernel_profile read 0 after it (the counters are kept).
 * Calls share their GPU's scratch array and keep nothing from one call to the
 * next; the library lock serialises calls within a process. Same algorithm,
 * parameters, results and errors as dance_vamana_build_resident. */
int dance_vamana_build_resident_noalloc(const void *d_data, int dtype, uint32_t num_points, uint32_t dim,
                                        uint32_t R, uint32_t L, uint32_t C, uint32_t STEPS, uint32_t *d_graph,
                                        uint32_t *d_degree);

/* Stitched build (reference: apps/utils/gpu_stitched_vamana_index.cpp,
 * label loop :276-341). For each label l in order 0..num_labels-1 with points
 * label_points[label_offsets[l] .. label_offsets[l+1]) (ascending ids), a
 * standard build over those points with R_small, L_small, C, STEPS; then
 * every local row is mapped to global ids and appended to its point's global
 * row: at most R_stitched leading entries of the local row, dropping invalid
 * local ids, self loops and ids the global row already holds. Rows of the
 * global graph have row_cap slots (INVALID-padded past the degree); row_cap
 * must hold every label of a point (labels x min(R_small, R_stitched)) and be
 * at most 256. label_medoids[l] is the global id of label l's medoid
 * (INVALID for a label without points). Label postings and medoids are host
 * arrays. Returns 0, or -1 with a message. The per-label builds run on
 * several streams at once (DANCE_STITCHED_WORKERS, default 8);
 * materialize_seconds and build_sum_seconds add up the per-label times, so
 * they can exceed total_seconds. */
typedef struct {
    double setup_seconds, materialize_seconds, build_sum_seconds, build_max_seconds, remap_seconds, total_seconds;
    uint64_t memberships, remap_invalid_local_ids, remap_self_loops, remap_duplicate_edges;
    uint32_t labels, label_npts_min, label_npts_max, row_cap;
    /* device memory in use (hipMemGetInfo: total - free, GiB, every process
     * on the GPU counted), the largest of the samples before the label loop,
     * after each label build and after the remap, as the reference's app
     * reports it (apps/utils/gpu_stitched_vamana_index.cpp:231-306) */
    double peak_gpu_mem_gb;
} DanceStitchedStats;

int dance_stitched_build(const void *h_data, int dtype, uint32_t num_points, uint32_t dim,
                         const uint32_t *label_offsets, const uint32_t *label_points, uint32_t num_labels,
                         uint32_t R_small, uint32_t L_small, uint32_t C, uint32_t STEPS, uint32_t R_stitched,
                         uint32_t row_cap, uint32_t *h_graph, uint32_t *h_degree, uint32_t *label_medoids);
/* The same with device rows (packed N x dim) and device outputs. */
int dance_stitched_build_resident(const void *d_data, int dtype, uint32_t num_points, uint32_t dim,
                                  const uint32_t *label_offsets, const uint32_t *label_points, uint32_t num_labels,
                                  uint32_t R_small, uint32_t L_small, uint32_t C, uint32_t STEPS,
                                  uint32_t R_stitched, uint32_t row_cap, uint32_t *d_graph, uint32_t *d_degree,
                                  uint32_t *label_medoids);
void dance_get_last_stitched_stats(DanceStitchedStats *stats);

/* Timings and counters of the last build on this process. */
void dance_get_last_kernel_profile(DanceKernelProfile *profile);

/* Selects the build profile at run time: "QUALITY" (default, fp32 storage),
 * "FAST_SMALL" (fp16 storage for float input), "PRO6000_100M" and
 * "FILTERED_PAPER" (fp16 + reverse heavy cap 256/384). Reference: CMake
 * DANCE_PROFILE, integrations/dance-diskann-78256bba.patch:2400-2462. The
 * DANCE_PROFILE environment variable sets the initial value. */
int dance_set_profile(const char *name);
const char *dance_get_profile(void);

/* ---- label-filtered build (gpu_vamana_filtered.h) extensions ---- */

/* Per-kernel timings (HIP events) and device-counted work of the last
 * filtered build. row_ms covers the fused union search, merge, label quota,
 * work distances and forward prune; csr_ms the exact reverse-CSR prune. */
typedef struct DanceFilteredProfile {
    double backbone_ms, task_search_ms, row_ms, reverse_ms, csr_ms, diagnostics_ms, total_ms;
    uint32_t rounds;
    uint32_t vector_bytes;
    uint64_t task_dist, union_dist, work_dist, prune_dist, csr_dist, csr_prune_dist;
    uint64_t merged_candidates, quota_dropped, reverse_edges, touched_rows, csr_candidates, long_lists;
    uint64_t out_edges, common_edges;
    /* largest CSR candidate list of a row (long lists: over 256 candidates) */
    uint64_t long_max_candidates;
    /* publish step (DISKANN_GPU_FILTERED_PUBLISH_DEGREE below R): kernel time,
     * distances, rows rebuilt from reverse sources, scratch entries of lists
     * over 256 candidates; publish_degree is the output graph's row width */
    double publish_ms;
    uint64_t publish_dist, publish_touched, publish_long_entries;
    uint32_t publish_degree, reserved0;
    /* per-label (task) and union-label searches: expansions (adjacency rows
     * read) and label-row reads of candidates that pass the signature filter */
    uint64_t task_expansions, task_label_reads, union_expansions, union_label_reads;
} DanceFilteredProfile;

/* The filtered build of gpu_vamana_filtered_build_{uint8,float} (reference:
 * src/gpu_vamana_filtered.cu:6511-7067) with the element type as a parameter
 * (DANCE_DTYPE_F32: searched as fp16; DANCE_DTYPE_U8; DANCE_DTYPE_F16: host
 * fp16 rows) and the number of canonical rounds (0..3; 3 is the reference,
 * 0 returns the random backbone). Used by the parity tests. */
int dance_filtered_build(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t L,
                         uint32_t filtered_L, uint32_t C, uint32_t STEPS, float alpha,
                         const uint32_t *point_label_offsets, const uint32_t *point_labels,
                         uint32_t total_label_count, const uint32_t *label_to_start_id, uint32_t num_labels,
                         uint32_t universal_label_id, uint32_t global_start_id, uint32_t rounds, uint32_t *h_graph,
                         uint32_t *h_degree);

/* Filtered build with the vectors resident in device memory (labels stay on
 * the host, as in the reference ABI) and device outputs; used by the bench. */
int dance_filtered_build_resident(const void *d_data, int dtype, uint32_t num_points, uint32_t dim, uint32_t R,
                                  uint32_t L, uint32_t filtered_L, uint32_t C, uint32_t STEPS, float alpha,
                                  const uint32_t *point_label_offsets, const uint32_t *point_labels,
                                  uint32_t total_label_count, const uint32_t *label_to_start_id,
                                  uint32_t num_labels, uint32_t universal_label_id, uint32_t global_start_id,
                                  uint32_t *d_graph, uint32_t *d_degree);

void dance_get_last_filtered_profile(DanceFilteredProfile *profile);

/* ---- query search over a built graph ---- */

/* Kernel time (HIP events) and device counters of the last search. */
typedef struct DanceSearchStats {
    double kernel_ms;
    uint64_t distances, expansions, capped_queries;
} DanceSearchStats;

/* Best-first search of num_queries query rows (host, same dtype and dim as
 * the base) over a graph (N x R rows, degree per row): DiskANN
 * search_memory_index semantics (reference counterpart; filtered start points
 * integrations/dance-diskann-78256bba.patch:20583-20600): a candidate list of
 * the L smallest (distance, id) seen, the closest unexpanded candidate is
 * expanded until none is left; returns the k best ids and canonical squared
 * distances per query in order (0xFFFFFFFF / FLT_MAX past the end). starts
 * holds 1 shared or num_queries entry points. With point_label_offsets /
 * point_labels / query_labels (all or none), only points carrying the query's
 * label are visited besides the start. 1 <= k <= 64, k <= L <= 1024 (the
 * reference's published sweeps run to L = 1000, REPRODUCIBILITY.md:44-52,
 * 96-104). Expansions are capped at 16 L + 1024 per query (capped_queries
 * counts hits). */
int dance_search(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, const uint32_t *h_graph,
                 const uint32_t *h_degree, uint32_t R, const uint32_t *starts, uint32_t num_starts,
                 const void *h_queries, uint32_t num_queries, uint32_t k, uint32_t L,
                 const uint32_t *point_label_offsets, const uint32_t *point_labels, const uint32_t *query_labels,
                 uint32_t *ids_out, float *dists_out);

/* Same with the base rows, graph and degrees resident in device memory. */
int dance_search_resident(const void *d_data, int dtype, uint32_t num_points, uint32_t dim, const uint32_t *d_graph,
                          const uint32_t *d_degree, uint32_t R, const uint32_t *starts, uint32_t num_starts,
                          const void *h_queries, uint32_t num_queries, uint32_t k, uint32_t L,
                          const uint32_t *point_label_offsets, const uint32_t *point_labels,
                          const uint32_t *query_labels, uint32_t *ids_out, float *dists_out);

/* dance_search with several entry points per query: query q starts from
 * starts[start_offsets[q] .. start_offsets[q + 1]) (start_offsets holds
 * num_queries + 1 non-decreasing entries from 0), all inserted into the
 * candidate list before the first expansion, without the label check; ids
 * >= num_points are skipped. This is DiskANN's filtered search seeded with a
 * label's start and its extra starts (the medoid list of
 * _labels_to_medoids.txt and DISKANN_FILTERED_SEARCH_EXTRA_STARTS,
 * integrations/dance-diskann-78256bba.patch:19780-19880; init_ids sorted and
 * deduplicated, :20583-20625). */
int dance_search_multistart(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, const uint32_t *h_graph,
                            const uint32_t *h_degree, uint32_t R, const uint32_t *start_offsets,
                            const uint32_t *starts, const void *h_queries, uint32_t num_queries, uint32_t k,
                            uint32_t L, const uint32_t *point_label_offsets, const uint32_t *point_labels,
                            const uint32_t *query_labels, uint32_t *ids_out, float *dists_out);
/* Same with the base rows, graph and degrees resident in device memory. */
int dance_search_multistart_resident(const void *d_data, int dtype, uint32_t num_points, uint32_t dim,
                                     const uint32_t *d_graph, const uint32_t *d_degree, uint32_t R,
                                     const uint32_t *start_offsets, const uint32_t *starts, const void *h_queries,
                                     uint32_t num_queries, uint32_t k, uint32_t L,
                                     const uint32_t *point_label_offsets, const uint32_t *point_labels,
                                     const uint32_t *query_labels, uint32_t *ids_out, float *dists_out);

void dance_get_last_search_stats(DanceSearchStats *stats);

/* ---- shard-graph merge (gpu_merge.h) ---- */

/* Counters and timings of the last merge_shards_gpu / dance_merge_shards call.
 * unique_edges counts distinct (source, target) pairs after self loops are
 * dropped; output_edges those kept under max_degree; long_segments the sources
 * whose edge list exceeded one wave's LDS sort and took the radix-sort path;
 * device_ms is HIP-event time of the device passes (expand, scan, rank, pack). */
typedef struct DanceMergeStats {
    uint64_t nnodes, replicated_nodes, input_edges, self_loops, unique_edges, output_edges;
    uint32_t min_degree, max_degree;
    uint64_t buckets, long_segments;
    uint32_t resident_shards, reserved0;
    double read_seconds, device_ms, write_seconds, total_seconds;
} DanceMergeStats;

/* C-ABI form of diskann::merge_shards_gpu (include/gpu_merge.h; reference
 * include/gpu_merge.h:8-12): the same files, arguments and return codes, with
 * C strings in place of std::string. */
int dance_merge_shards(const char *vamana_prefix, const char *vamana_suffix, const char *idmaps_prefix,
                       const char *idmaps_suffix, uint64_t nshards, uint32_t max_degree, const char *output_vamana,
                       const char *medoids_file);

void dance_merge_get_last_stats(DanceMergeStats *stats);

/* Shard assignment of the sharded build (DiskANN's
 * shard_data_into_clusters_only_ids and its k-means assignment step, upstream
 * partition.cpp, called from build_merged_vamana_index,
 * integrations/dance-diskann-78256bba.patch:1212-1260): for each of
 * num_points host rows (dtype DANCE_DTYPE_F32 or DANCE_DTYPE_U8, dim <= 255)
 * the k_base (1..min(8, num_centers)) nearest of num_centers fp32 centers,
 * nearest first, into h_assign (num_points x k_base). Distances are squared
 * L2 accumulated in fp64 in dimension order (fma per dimension); ties go to
 * the lower center index; a point whose distances are all NaN gets
 * 0xFFFFFFFF. Returns 0, or -1 on invalid arguments or a HIP error. */
int dance_partition_assign(const void *h_data, int dtype, uint64_t num_points, uint32_t dim, const float *h_centers,
                           uint32_t num_centers, uint32_t k_base, uint32_t *h_assign);

/* Sizes in bytes of the structs this library fills, in the order
 * GPUVamanaStats, DanceKernelProfile, GPUFilteredVamanaStats,
 * DanceFilteredProfile, DanceSearchStats, DanceMergeStats; writes
 * min(count, 6) entries and returns 6. Bindings compare them with their own
 * layouts before any call that writes a struct. */
uint32_t dance_struct_sizes(uint64_t *sizes, uint32_t count);

/* ---- stage hooks (host buffers), used by the parity tests ---- */

/* Canonical squared-L2 distances d(a[i], b[i]) (reference distance family,
 * src/gpu_vamana_vnew2.cu:215-423). */
int dance_stage_distances(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, const uint32_t *a,
                          const uint32_t *b, uint64_t n, float *out);

/* The search's quantized distance bound on explicit pairs (no counterpart in
 * the reference; it only skips work): flags[i] = 1 when the bound proves
 * dist(a[i], b[i]) >= T[i]. fp32/fp16 rows of <= 112 dims; -1 otherwise. */
int dance_stage_qbound(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, const uint32_t *a,
                       const uint32_t *b, const float *T, uint64_t n, uint32_t *flags);

/* The online insert's occlusion-pair bounds on explicit pairs (no
 * counterpart in the reference; they only skip work), with x = a[i], y = b[i]
 * and T0[i] = d_px: out[i] = 1 when the code rows prove
 * fl(alpha * dist(x, y)) <= T0[i], 2 when they prove it > T0[i], 0 when
 * neither. fp32/fp16 rows of <= 112 dims; -1 otherwise. */
int dance_stage_insert_bound(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, const uint32_t *a,
                             const uint32_t *b, const float *T0, float alpha, uint64_t n, uint32_t *out);

/* medoid_score_kernel_warp + host top-1 (src/gpu_vamana_vnew2.cu:1032-1064, 2359-2479).
 * scores/cands: min(1024, N) entries. */
int dance_stage_medoid(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, float *scores,
                       uint32_t *cands, uint32_t *medoid);

/* init_random_graph (src/gpu_vamana_vnew2.cu:1066-1117). */
int dance_stage_init(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t C,
                     uint32_t *cur, uint32_t *deg_cur, uint32_t *work, uint32_t *deg_work, float *wd);

/* One search + online-insert pass over all vertices
 * (search_prune_kernel_shared, src/gpu_vamana_vnew2.cu:1119-1439). In/out graph state. */
int dance_stage_search(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t L,
                       uint32_t C, uint32_t steps, float alpha, uint32_t start, uint32_t *cur, uint32_t *deg_cur,
                       uint32_t *work, uint32_t *deg_work, float *wd);

/* Reverse CSR + merge (reverse_count/fill_csr_kernel + reverse_merge_csr_kernel,
 * src/gpu_vamana_vnew2.cu:1604-1661, 1722-1814). offsets (N+1) and ids (N*R)
 * receive the canonical CSR when non-null. Precondition, as in every work row
 * the build produces: the stored distance of each valid entry among the first
 * R is the canonical distance of the row's vertex to it (the merge reads it
 * instead of recomputing the symmetric distance). */
int dance_stage_reverse_merge(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, uint32_t R,
                              uint32_t C, uint32_t *work, uint32_t *deg_work, float *wd, uint32_t heavy_threshold,
                              uint32_t heavy_sample, uint32_t *offsets, uint32_t *ids);

/* RobustPrune + degree fill (final_prune_kernel_shared, src/gpu_vamana_vnew2.cu:1893-2147). */
int dance_stage_prune(const void *h_data, int dtype, uint32_t num_points, uint32_t dim, uint32_t R, uint32_t C,
                      uint32_t min_degree, float alpha, uint32_t *work, uint32_t *deg_work, float *wd,
                      uint32_t *cur, uint32_t *deg_cur);

/* Stable radix sort of (key, value) pairs on the low `key_bits` bits
 * (replaces thrust/CUB primitives of the reference). */
int dance_stage_sort_pairs(const uint32_t *keys, const uint32_t *vals, uint64_t n, uint32_t key_bits,
                           uint32_t *out_keys, uint32_t *out_vals);

/* Exclusive prefix sum of n uint32 values (replaces thrust::inclusive_scan,
 * src/gpu_vamana_vnew2.cu:2576-2577). */
int dance_stage_scan(const uint32_t *in, uint64_t n, uint32_t *out);

/* ---- synthetic workloads (host, multithreaded, deterministic) ---- */

/* Gaussian-mixture vectors: centers ~ N(0, I) (num_centers = 0: pure N(0, I)),
 * x = c_k + sigma * eps, optionally L2-normalised. stream selects an
 * independent sub-stream (0 = base, 1 = queries, ...). fp32 rows. */
int dance_synth_f32(uint64_t seed, uint32_t stream, uint32_t num_points, uint32_t dim, uint32_t num_centers,
                    float sigma, int normalize, float *out);

/* uint8 rows clip(round(64 + 24 z), 0, 255) of a Gaussian mixture z. */
int dance_synth_u8(uint64_t seed, uint32_t stream, uint32_t num_points, uint32_t dim, uint32_t num_centers,
                   float sigma, uint8_t *out);

#ifdef __cplusplus
}
#endif

#endif
