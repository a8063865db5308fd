"""dance_amd: MI355X-native (gfx950) GPU Vamana graph construction.

Host-side Python mirror of the reference's builder interfaces
(/root/reference/include/gpu_vamana_builder.h, gpu_vamana_filtered.h; the
filtered build's helpers live in dance_amd.filtered). All device work runs in
libdance_hip.so (hand-written HIP kernels); this module only marshals numpy
arrays and device pointers across the C ABI. There is no CPU fallback: if the
library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# DANCE_HIP_LIB points at another build of the same library (e.g. one compiled
# with DANCE_SEARCH_TIMING=1); default is the in-tree build.
LIB_PATH = os.environ.get("DANCE_HIP_LIB") or os.path.join(HERE, "libdance_hip.so")

DTYPE_F32, DTYPE_U8, DTYPE_F16 = 0, 1, 2
INVALID = 0xFFFFFFFF

_u32p = C.POINTER(C.c_uint32)
_f32p = C.POINTER(C.c_float)


class GPUVamanaStats(C.Structure):
    """Layout of GPUVamanaStats (reference include/gpu_vamana_builder.h:11-28)."""

    _fields_ = [
        ("medoid_seconds", C.c_double),
        ("h2d_seconds", C.c_double),
        ("search_online_insert_seconds", C.c_double),
        ("reverse_seconds", C.c_double),
        ("final_prune_seconds", C.c_double),
        ("d2h_seconds", C.c_double),
        ("gpu_build_seconds", C.c_double),
        ("distance_computations", C.c_uint64),
        ("online_insert_attempts", C.c_uint64),
        ("online_insert_mutations", C.c_uint64),
        ("reverse_candidate_overflows", C.c_uint64),
        ("reverse_proposals", C.c_uint64),
        ("reverse_touched_rows", C.c_uint64),
        ("reverse_csr_seconds", C.c_double),
        ("selective_active_nodes", C.c_uint32),
    ]


# DANCE_MAX_ITERS of include/dance_hip.h: length of the per-iteration arrays
MAX_ITERS = 8


class DanceKernelProfile(C.Structure):
    _fields_ = [
        ("medoid_ms", C.c_double), ("init_ms", C.c_double), ("search_ms", C.c_double),
        ("reverse_ms", C.c_double), ("merge_ms", C.c_double), ("prune_ms", C.c_double),
        ("total_ms", C.c_double),
        ("iterations", C.c_uint32), ("vector_bytes", C.c_uint32),
        ("search_dist", C.c_uint64), ("insert_dist", C.c_uint64), ("expansions", C.c_uint64),
        ("vis_skips", C.c_uint64), ("merge_dist", C.c_uint64), ("prune_dist", C.c_uint64),
        ("reverse_edges", C.c_uint64), ("touched_rows", C.c_uint64),
        ("search_bytes", C.c_double), ("merge_bytes", C.c_double), ("prune_bytes", C.c_double),
        ("reverse_bytes", C.c_double),
        ("cyc_select", C.c_uint64), ("cyc_insert", C.c_uint64), ("cyc_dist", C.c_uint64),
        ("cyc_pool", C.c_uint64), ("cyc_seed", C.c_uint64), ("cyc_total", C.c_uint64),
        ("bound_checks", C.c_uint64), ("bound_skips", C.c_uint64),
        ("prune_bound_checks", C.c_uint64), ("prune_bound_skips", C.c_uint64),
        ("search_iter_ms", C.c_double * MAX_ITERS), ("prune_iter_ms", C.c_double * MAX_ITERS),
        ("search_dist_iter", C.c_uint64 * MAX_ITERS), ("insert_dist_iter", C.c_uint64 * MAX_ITERS),
        ("expansions_iter", C.c_uint64 * MAX_ITERS), ("bound_checks_iter", C.c_uint64 * MAX_ITERS),
        ("bound_skips_iter", C.c_uint64 * MAX_ITERS), ("merge_dist_iter", C.c_uint64 * MAX_ITERS),
        ("prune_dist_iter", C.c_uint64 * MAX_ITERS), ("prune_bound_checks_iter", C.c_uint64 * MAX_ITERS),
        ("prune_bound_skips_iter", C.c_uint64 * MAX_ITERS),
        ("search_bytes_iter", C.c_double * MAX_ITERS), ("prune_bytes_iter", C.c_double * MAX_ITERS),
        ("prune_rounds", C.c_uint64), ("prune_exact_rounds", C.c_uint64),
        ("cyc_prune_rank", C.c_uint64), ("cyc_prune_gram", C.c_uint64), ("cyc_prune_rounds", C.c_uint64),
        ("cyc_prune_fill", C.c_uint64),
        ("insert_bound_checks", C.c_uint64), ("insert_bound_skips", C.c_uint64),
        ("insert_bound_checks_iter", C.c_uint64 * MAX_ITERS), ("insert_bound_skips_iter", C.c_uint64 * MAX_ITERS),
    ]


_FILTERED_STATS_FIELDS = (
    [(n, C.c_double) for n in (
        "gpu_build_seconds", "label_h2d_seconds", "graph_build_seconds", "diagnostics_seconds", "d2h_seconds",
        "peak_gpu_mem_gb", "backbone_seconds", "task_generation_seconds", "filtered_search_seconds",
        "ordinary_search_seconds", "merge_seconds", "forward_prune_seconds", "csr_reverse_seconds",
        "reverse_prune_seconds", "compaction_seconds")]
    + [(n, C.c_uint64) for n in (
        "filtered_search_distance_count", "unfiltered_search_distance_count", "label_check_count",
        "label_reject_count", "filtered_candidate_count", "unfiltered_candidate_count", "merged_candidate_count",
        "active_rows", "original_neighbor_count", "filtered_seed_count", "filtered_visited_count",
        "filtered_visited_reserved_count", "filtered_top_reserved_count", "bridge_reserved_count",
        "unfiltered_reserved_count", "filtered_reserved_count", "label_occlusion_blocked_count",
        "geometry_occluded_count", "candidate_rejected_by_label_count", "refill_count",
        "filtered_prune_reject_count", "universal_label_pass_count", "final_prune_rows", "reverse_edges",
        "reverse_touched_rows", "filtered_reverse_edges", "filtered_reverse_touched_rows",
        "filtered_reverse_candidates_kept", "filtered_reverse_pruned_rows")]
    + [(n, C.c_double) for n in (
        "avg_common_label_out_degree", "common_label_degree_before_avg", "common_label_degree_after_avg",
        "active_rows_frac")]
    + [(n, C.c_uint32) for n in (
        "low_common_label_degree_count", "low_common_before", "low_common_after", "out_degree_min",
        "out_degree_max")]
    + [("out_degree_avg", C.c_double)]
    + [(n, C.c_uint32) for n in (
        "common_label_degree_min", "common_label_degree_max", "invalid_neighbor_count", "self_loop_count")]
    + [("prune_output_degree_avg", C.c_double)]
    + [(n, C.c_uint32) for n in ("filtered_seed_source", "semantic_stage", "semantic_complete")]
)


class GPUFilteredVamanaStats(C.Structure):
    """Layout of GPUFilteredVamanaStats (reference include/gpu_vamana_filtered.h:11-77)."""

    _fields_ = _FILTERED_STATS_FIELDS


class DanceFilteredProfile(C.Structure):
    _fields_ = (
        [(n, C.c_double) for n in ("backbone_ms", "task_search_ms", "row_ms", "reverse_ms", "csr_ms",
                                   "diagnostics_ms", "total_ms")]
        + [("rounds", C.c_uint32), ("vector_bytes", C.c_uint32)]
        + [(n, C.c_uint64) for n in ("task_dist", "union_dist", "work_dist", "prune_dist", "csr_dist",
                                     "csr_prune_dist", "merged_candidates", "quota_dropped", "reverse_edges",
                                     "touched_rows", "csr_candidates", "long_lists", "out_edges",
                                     "common_edges", "long_max_candidates")]
        + [("publish_ms", C.c_double)]
        + [(n, C.c_uint64) for n in ("publish_dist", "publish_touched", "publish_long_entries")]
        + [("publish_degree", C.c_uint32), ("reserved0", C.c_uint32)]
        + [(n, C.c_uint64) for n in ("task_expansions", "task_label_reads", "union_expansions",
                                     "union_label_reads")]
    )


class DanceSearchStats(C.Structure):
    _fields_ = [("kernel_ms", C.c_double), ("distances", C.c_uint64), ("expansions", C.c_uint64),
                ("capped_queries", C.c_uint64)]


class DanceStitchedStats(C.Structure):
    _fields_ = ([(n, C.c_double) for n in ("setup_seconds", "materialize_seconds", "build_sum_seconds",
                                           "build_max_seconds", "remap_seconds", "total_seconds")]
                + [(n, C.c_uint64) for n in ("memberships", "remap_invalid_local_ids", "remap_self_loops",
                                             "remap_duplicate_edges")]
                + [(n, C.c_uint32) for n in ("labels", "label_npts_min", "label_npts_max", "row_cap")]
                + [("peak_gpu_mem_gb", C.c_double)])


def struct_dict(s: C.Structure) -> dict:
    out = {}
    for name, _ in s._fields_:
        v = getattr(s, name)
        out[name] = list(v) if isinstance(v, C.Array) else v
    return out


# Every symbol the C ABI exports (include/*.h). Tests check the library
# exports exactly these.
EXPORTS = [
    "gpu_vamana_build", "gpu_vamana_build_float",
    "gpu_vamana_vnew2_build", "gpu_vamana_vnew2_build_float",
    "gpu_vamana_vnew2_build_device", "gpu_vamana_vnew2_build_device_float",
    "gpu_vamana_get_last_medoid", "gpu_vamana_get_last_stats",
    "gpu_vamana_vnew2_get_last_medoid", "gpu_vamana_vnew2_get_last_stats",
    "dance_vamana_build_resident", "dance_vamana_build_resident_noalloc", "dance_get_last_kernel_profile",
    "dance_set_profile", "dance_get_profile",
    "dance_stage_distances", "dance_stage_qbound", "dance_stage_insert_bound", "dance_stage_medoid",
    "dance_stage_init", "dance_stage_search",
    "dance_stage_reverse_merge", "dance_stage_prune", "dance_stage_sort_pairs", "dance_stage_scan",
    "dance_synth_f32", "dance_synth_u8",
    "gpu_vamana_filtered_build_uint8", "gpu_vamana_filtered_build_float", "gpu_vamana_filtered_get_last_stats",
    "dance_filtered_build", "dance_filtered_build_resident", "dance_get_last_filtered_profile",
    "dance_search", "dance_search_resident", "dance_search_multistart", "dance_search_multistart_resident",
    "dance_get_last_search_stats",
    "dance_merge_shards", "dance_merge_get_last_stats", "dance_struct_sizes",
    "dance_partition_assign",
    "dance_stitched_build", "dance_stitched_build_resident", "dance_get_last_stitched_stats",
]

class DanceMergeStats(C.Structure):
    _fields_ = [
        ("nnodes", C.c_uint64), ("replicated_nodes", C.c_uint64), ("input_edges", C.c_uint64),
        ("self_loops", C.c_uint64), ("unique_edges", C.c_uint64), ("output_edges", C.c_uint64),
        ("min_degree", C.c_uint32), ("max_degree", C.c_uint32),
        ("buckets", C.c_uint64), ("long_segments", C.c_uint64),
        ("resident_shards", C.c_uint32), ("reserved0", C.c_uint32),
        ("read_seconds", C.c_double), ("device_ms", C.c_double), ("write_seconds", C.c_double),
        ("total_seconds", C.c_double),
    ]



_LIB = None


def _check_struct_sizes(L) -> None:
    """The library writes these structs into memory this module allocates:
    a layout mismatch (a library built from other headers) must fail here,
    before it can overrun a buffer."""
    mine = [GPUVamanaStats, DanceKernelProfile, GPUFilteredVamanaStats, DanceFilteredProfile, DanceSearchStats,
            DanceMergeStats, DanceStitchedStats]
    L.dance_struct_sizes.argtypes = [C.POINTER(C.c_uint64), C.c_uint32]
    L.dance_struct_sizes.restype = C.c_uint32
    got = (C.c_uint64 * len(mine))()
    L.dance_struct_sizes(got, len(mine))
    for cls, size in zip(mine, got):
        if C.sizeof(cls) != size:
            raise RuntimeError(f"{LIB_PATH}: {cls.__name__} is {size} bytes in the library and {C.sizeof(cls)} "
                               "here; rebuild the library (python -m dance_amd.build)")


def lib() -> C.CDLL:
    """Loads libdance_hip.so; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `python -m dance_amd.build` "
                               "(or __graft_entry__.build()) first")
        # PyTorch-ROCm ships its own HIP runtime (torch/lib/libamdhip64.so,
        # requested by that unversioned name). If this library loaded the
        # system runtime (libamdhip64.so.7) first, a later torch import would
        # start a second HIP/HSA runtime in the process, which then finds no
        # GPU. Loading torch first makes the library bind to torch's copy
        # (same soname), so one runtime serves both and torch device pointers
        # are valid here.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        _check_struct_sizes(L)
        u32, f32, vp, i32 = C.c_uint32, C.c_float, C.c_void_p, C.c_int
        build_args = [vp, u32, u32, u32, u32, u32, u32, _u32p, _u32p]
        for name in ("gpu_vamana_build", "gpu_vamana_build_float", "gpu_vamana_vnew2_build",
                     "gpu_vamana_vnew2_build_float"):
            getattr(L, name).argtypes = build_args
            getattr(L, name).restype = i32
        for name in ("gpu_vamana_vnew2_build_device", "gpu_vamana_vnew2_build_device_float"):
            getattr(L, name).argtypes = [vp, u32, u32, u32, u32, u32, u32, C.POINTER(vp),
                                         C.POINTER(vp), C.POINTER(vp)]
            getattr(L, name).restype = i32
        for name in ("gpu_vamana_get_last_medoid", "gpu_vamana_vnew2_get_last_medoid"):
            getattr(L, name).restype = u32
            getattr(L, name).argtypes = []
        for name in ("gpu_vamana_get_last_stats", "gpu_vamana_vnew2_get_last_stats"):
            getattr(L, name).argtypes = [C.POINTER(GPUVamanaStats)]
            getattr(L, name).restype = None
        for name in ("dance_vamana_build_resident", "dance_vamana_build_resident_noalloc"):
            getattr(L, name).argtypes = [vp, i32, u32, u32, u32, u32, u32, u32, vp, vp]
            getattr(L, name).restype = i32
        L.dance_get_last_kernel_profile.argtypes = [C.POINTER(DanceKernelProfile)]
        L.dance_get_last_kernel_profile.restype = None
        L.dance_set_profile.argtypes = [C.c_char_p]
        L.dance_set_profile.restype = i32
        L.dance_get_profile.argtypes = []
        L.dance_get_profile.restype = C.c_char_p
        L.dance_stage_distances.argtypes = [vp, i32, u32, u32, _u32p, _u32p, C.c_uint64, _f32p]
        L.dance_stage_qbound.argtypes = [vp, i32, u32, u32, _u32p, _u32p, _f32p, C.c_uint64, _u32p]
        L.dance_stage_insert_bound.argtypes = [vp, i32, u32, u32, _u32p, _u32p, _f32p, f32, C.c_uint64, _u32p]
        L.dance_stage_medoid.argtypes = [vp, i32, u32, u32, _f32p, _u32p, _u32p]
        L.dance_stage_init.argtypes = [vp, i32, u32, u32, u32, u32, _u32p, _u32p, _u32p, _u32p, _f32p]
        L.dance_stage_search.argtypes = [vp, i32, u32, u32, u32, u32, u32, u32, f32, u32,
                                         _u32p, _u32p, _u32p, _u32p, _f32p]
        L.dance_stage_reverse_merge.argtypes = [vp, i32, u32, u32, u32, u32, _u32p, _u32p, _f32p,
                                                u32, u32, _u32p, _u32p]
        L.dance_stage_prune.argtypes = [vp, i32, u32, u32, u32, u32, u32, f32, _u32p, _u32p, _f32p,
                                        _u32p, _u32p]
        L.dance_stage_sort_pairs.argtypes = [_u32p, _u32p, C.c_uint64, u32, _u32p, _u32p]
        L.dance_stage_scan.argtypes = [_u32p, C.c_uint64, _u32p]
        for name in ("dance_stage_distances", "dance_stage_qbound", "dance_stage_insert_bound", "dance_stage_medoid",
                     "dance_stage_init", "dance_stage_search", "dance_stage_reverse_merge", "dance_stage_prune",
                     "dance_stage_sort_pairs", "dance_stage_scan"):
            getattr(L, name).restype = i32
        L.dance_synth_f32.argtypes = [C.c_uint64, u32, u32, u32, u32, f32, i32, _f32p]
        L.dance_synth_f32.restype = i32
        L.dance_synth_u8.argtypes = [C.c_uint64, u32, u32, u32, u32, f32, C.POINTER(C.c_uint8)]
        L.dance_synth_u8.restype = i32
        labels_args = [_u32p, _u32p, u32, _u32p, u32, u32, u32]
        for name in ("gpu_vamana_filtered_build_uint8", "gpu_vamana_filtered_build_float"):
            getattr(L, name).argtypes = ([vp, u32, u32, u32, u32, u32, u32, u32, f32] + labels_args
                                         + [_u32p, _u32p, u32, _u32p, _u32p])
            getattr(L, name).restype = i32
        L.gpu_vamana_filtered_get_last_stats.argtypes = [C.POINTER(GPUFilteredVamanaStats)]
        L.gpu_vamana_filtered_get_last_stats.restype = None
        L.dance_filtered_build.argtypes = ([vp, i32, u32, u32, u32, u32, u32, u32, u32, f32] + labels_args
                                           + [u32, _u32p, _u32p])
        L.dance_filtered_build.restype = i32
        L.dance_filtered_build_resident.argtypes = ([vp, i32, u32, u32, u32, u32, u32, u32, u32, f32] + labels_args
                                                    + [vp, vp])
        L.dance_filtered_build_resident.restype = i32
        L.dance_get_last_filtered_profile.argtypes = [C.POINTER(DanceFilteredProfile)]
        L.dance_get_last_filtered_profile.restype = None
        search_args = [vp, i32, u32, u32, vp, vp, u32, _u32p, u32, vp, u32, u32, u32, vp, vp, vp, _u32p, _f32p]
        for name in ("dance_search", "dance_search_resident"):
            getattr(L, name).argtypes = search_args
            getattr(L, name).restype = i32
        multi_args = [vp, i32, u32, u32, vp, vp, u32, _u32p, _u32p, vp, u32, u32, u32, vp, vp, vp, _u32p, _f32p]
        for name in ("dance_search_multistart", "dance_search_multistart_resident"):
            getattr(L, name).argtypes = multi_args
            getattr(L, name).restype = i32
        L.dance_get_last_search_stats.argtypes = [C.POINTER(DanceSearchStats)]
        L.dance_get_last_search_stats.restype = None
        for name in ("dance_stitched_build", "dance_stitched_build_resident"):
            getattr(L, name).argtypes = [vp, i32, u32, u32, _u32p, _u32p, u32, u32, u32, u32, u32, u32, u32,
                                         vp, vp, _u32p]
            getattr(L, name).restype = i32
        L.dance_get_last_stitched_stats.argtypes = [C.POINTER(DanceStitchedStats)]
        L.dance_get_last_stitched_stats.restype = None
        _LIB = L
    return _LIB


def _p(a: np.ndarray, ctype):
    return a.ctypes.data_as(C.POINTER(ctype))


def dtype_code(arr: np.ndarray) -> int:
    if arr.dtype == np.float32:
        return DTYPE_F32
    if arr.dtype == np.uint8:
        return DTYPE_U8
    if arr.dtype == np.float16:
        return DTYPE_F16
    raise TypeError(f"unsupported vector dtype {arr.dtype}")


class BuildError(RuntimeError):
    pass


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise BuildError(f"{what} failed with return code {rc}")


@dataclass
class BuildResult:
    graph: np.ndarray   # N x R uint32, rows padded with INVALID after the degree
    degree: np.ndarray  # N uint32
    medoid: int
    stats: dict
    kernel_profile: dict


def set_profile(name: str) -> None:
    _check(lib().dance_set_profile(name.encode()), f"dance_set_profile({name})")


def get_profile() -> str:
    return lib().dance_get_profile().decode()


def last_kernel_profile() -> dict:
    """DanceKernelProfile of the last standard build; the per-iteration
    lists hold one entry per iteration the build ran."""
    p = DanceKernelProfile()
    lib().dance_get_last_kernel_profile(C.byref(p))
    out = struct_dict(p)
    n = int(out["iterations"])
    for k, v in out.items():
        if k.endswith(("_iter", "_iter_ms")):
            out[k] = v[:n]
    return out


def last_stats(entry: str = "vnew2") -> dict:
    """GPUVamanaStats of the last vnew2 build, or of the last v8 build."""
    s = GPUVamanaStats()
    getter = lib().gpu_vamana_get_last_stats if entry == "v8" else lib().gpu_vamana_vnew2_get_last_stats
    getter(C.byref(s))
    return struct_dict(s)


def last_medoid(entry: str = "vnew2") -> int:
    getter = lib().gpu_vamana_get_last_medoid if entry == "v8" else lib().gpu_vamana_vnew2_get_last_medoid
    return int(getter())


def vamana_build(data: np.ndarray, R: int = 64, L: int = 100, C_: int = 80, STEPS: int = 64,
                 entry: str = "vnew2") -> BuildResult:
    """gpu_vamana_vnew2_build[_float] (entry "vnew2") or the v8 builder's
    gpu_vamana_build[_float] (entry "v8") on host vectors (uint8 or float32)."""
    if entry not in ("vnew2", "v8"):
        raise ValueError(f"unknown builder entry {entry!r}")
    data = np.ascontiguousarray(data)
    if data.ndim != 2:
        raise ValueError("data must be N x dim")
    N, dim = data.shape
    graph = np.empty((N, R), dtype=np.uint32)
    degree = np.empty(N, dtype=np.uint32)
    L_ = lib()
    if data.dtype == np.float32:
        fn = L_.gpu_vamana_vnew2_build_float if entry == "vnew2" else L_.gpu_vamana_build_float
    elif data.dtype == np.uint8:
        fn = L_.gpu_vamana_vnew2_build if entry == "vnew2" else L_.gpu_vamana_build
    else:
        raise TypeError("vamana_build takes uint8 or float32 vectors")
    rc = fn(data.ctypes.data, N, dim, R, L, C_, STEPS, _p(graph, C.c_uint32), _p(degree, C.c_uint32))
    _check(rc, "gpu_vamana_vnew2_build" if entry == "vnew2" else "gpu_vamana_build")
    return BuildResult(graph, degree, last_medoid(entry), last_stats(entry), last_kernel_profile())


def vamana_build_resident(d_data: int, dtype: int, N: int, dim: int, R: int, L: int, C_: int, STEPS: int,
                          d_graph: int, d_degree: int) -> None:
    """dance_vamana_build_resident on device pointers (e.g. torch tensor data_ptr())."""
    _check(lib().dance_vamana_build_resident(d_data, dtype, N, dim, R, L, C_, STEPS, d_graph, d_degree),
           "dance_vamana_build_resident")


def vamana_build_resident_noalloc(d_data: int, dtype: int, N: int, dim: int, R: int, L: int, C_: int, STEPS: int,
                                  d_graph: int, d_degree: int) -> None:
    """dance_vamana_build_resident_noalloc: the same build with every device
    buffer taken from the library's per-GPU scratch array (no allocation)."""
    _check(lib().dance_vamana_build_resident_noalloc(d_data, dtype, N, dim, R, L, C_, STEPS, d_graph, d_degree),
           "dance_vamana_build_resident_noalloc")


# ---------------------------------------------------------------- stage hooks

def stage_distances(data: np.ndarray, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    data = np.ascontiguousarray(data)
    a = np.ascontiguousarray(a, dtype=np.uint32)
    b = np.ascontiguousarray(b, dtype=np.uint32)
    out = np.empty(a.shape[0], dtype=np.float32)
    _check(lib().dance_stage_distances(data.ctypes.data, dtype_code(data), data.shape[0], data.shape[1],
                                       _p(a, C.c_uint32), _p(b, C.c_uint32), a.shape[0],
                                       _p(out, C.c_float)), "dance_stage_distances")
    return out


def stage_qbound(data: np.ndarray, a: np.ndarray, b: np.ndarray, T: np.ndarray) -> np.ndarray:
    """Flags of the search's quantized bound: 1 where it proves dist(a, b) >= T."""
    data = np.ascontiguousarray(data)
    a = np.ascontiguousarray(a, dtype=np.uint32)
    b = np.ascontiguousarray(b, dtype=np.uint32)
    T = np.ascontiguousarray(T, dtype=np.float32)
    out = np.empty(a.shape[0], dtype=np.uint32)
    _check(lib().dance_stage_qbound(data.ctypes.data, dtype_code(data), data.shape[0], data.shape[1],
                                    _p(a, C.c_uint32), _p(b, C.c_uint32), _p(T, C.c_float), a.shape[0],
                                    _p(out, C.c_uint32)), "dance_stage_qbound")
    return out


def stage_insert_bound(data: np.ndarray, a: np.ndarray, b: np.ndarray, T0: np.ndarray, alpha: float) -> np.ndarray:
    """The online insert's occlusion-pair bounds (x = a, y = b, T0 = d_px):
    1 where the code rows prove fl(alpha * dist) <= T0, 2 where they prove
    fl(alpha * dist) > T0, 0 where the pair is left to the exact distance."""
    data = np.ascontiguousarray(data)
    a = np.ascontiguousarray(a, dtype=np.uint32)
    b = np.ascontiguousarray(b, dtype=np.uint32)
    T0 = np.ascontiguousarray(T0, dtype=np.float32)
    out = np.empty(a.shape[0], dtype=np.uint32)
    _check(lib().dance_stage_insert_bound(data.ctypes.data, dtype_code(data), data.shape[0], data.shape[1],
                                          _p(a, C.c_uint32), _p(b, C.c_uint32), _p(T0, C.c_float), float(alpha),
                                          a.shape[0], _p(out, C.c_uint32)), "dance_stage_insert_bound")
    return out


def stage_medoid(data: np.ndarray):
    data = np.ascontiguousarray(data)
    N = data.shape[0]
    nc = min(1024, N)
    scores = np.empty(nc, dtype=np.float32)
    cands = np.empty(nc, dtype=np.uint32)
    med = np.zeros(1, dtype=np.uint32)
    _check(lib().dance_stage_medoid(data.ctypes.data, dtype_code(data), N, data.shape[1],
                                    _p(scores, C.c_float), _p(cands, C.c_uint32), _p(med, C.c_uint32)),
           "dance_stage_medoid")
    return int(med[0]), scores, cands


@dataclass
class GraphState:
    cur: np.ndarray
    deg_cur: np.ndarray
    work: np.ndarray
    deg_work: np.ndarray
    wd: np.ndarray

    def copy(self) -> "GraphState":
        return GraphState(self.cur.copy(), self.deg_cur.copy(), self.work.copy(), self.deg_work.copy(),
                          self.wd.copy())

    @staticmethod
    def empty(N: int, R: int, C_: int) -> "GraphState":
        return GraphState(np.full((N, R), INVALID, np.uint32), np.zeros(N, np.uint32),
                          np.full((N, C_), INVALID, np.uint32), np.zeros(N, np.uint32),
                          np.full((N, C_), np.finfo(np.float32).max, np.float32))


def _gs_ptrs(g: GraphState):
    return (_p(g.cur, C.c_uint32), _p(g.deg_cur, C.c_uint32), _p(g.work, C.c_uint32),
            _p(g.deg_work, C.c_uint32), _p(g.wd, C.c_float))


def stage_init(data: np.ndarray, R: int, C_: int) -> GraphState:
    data = np.ascontiguousarray(data)
    g = GraphState.empty(data.shape[0], R, C_)
    _check(lib().dance_stage_init(data.ctypes.data, dtype_code(data), data.shape[0], data.shape[1], R, C_,
                                  *_gs_ptrs(g)), "dance_stage_init")
    return g


def stage_search(data: np.ndarray, g: GraphState, L: int, steps: int, alpha: float, start: int) -> GraphState:
    data = np.ascontiguousarray(data)
    g = g.copy()
    N, R = g.cur.shape
    _check(lib().dance_stage_search(data.ctypes.data, dtype_code(data), N, data.shape[1], R, L,
                                    g.work.shape[1], steps, alpha, start, *_gs_ptrs(g)), "dance_stage_search")
    return g


def stage_reverse_merge(data: np.ndarray, g: GraphState, heavy_threshold: int = 0, heavy_sample: int = 0):
    data = np.ascontiguousarray(data)
    g = g.copy()
    N, R = g.cur.shape
    offsets = np.zeros(N + 1, dtype=np.uint32)
    ids = np.zeros(N * R, dtype=np.uint32)
    _check(lib().dance_stage_reverse_merge(data.ctypes.data, dtype_code(data), N, data.shape[1], R,
                                           g.work.shape[1], _p(g.work, C.c_uint32), _p(g.deg_work, C.c_uint32),
                                           _p(g.wd, C.c_float), heavy_threshold, heavy_sample,
                                           _p(offsets, C.c_uint32), _p(ids, C.c_uint32)),
           "dance_stage_reverse_merge")
    return g, offsets, ids[: offsets[-1]]


def stage_prune(data: np.ndarray, g: GraphState, min_degree: int, alpha: float) -> GraphState:
    data = np.ascontiguousarray(data)
    g = g.copy()
    N, R = g.cur.shape
    _check(lib().dance_stage_prune(data.ctypes.data, dtype_code(data), N, data.shape[1], R, g.work.shape[1],
                                   min_degree, alpha, _p(g.work, C.c_uint32), _p(g.deg_work, C.c_uint32),
                                   _p(g.wd, C.c_float), _p(g.cur, C.c_uint32), _p(g.deg_cur, C.c_uint32)),
           "dance_stage_prune")
    return g


def stage_sort_pairs(keys: np.ndarray, vals: np.ndarray, key_bits: int):
    keys = np.ascontiguousarray(keys, dtype=np.uint32)
    vals = np.ascontiguousarray(vals, dtype=np.uint32)
    ok = np.empty_like(keys)
    ov = np.empty_like(vals)
    _check(lib().dance_stage_sort_pairs(_p(keys, C.c_uint32), _p(vals, C.c_uint32), keys.shape[0], key_bits,
                                        _p(ok, C.c_uint32), _p(ov, C.c_uint32)), "dance_stage_sort_pairs")
    return ok, ov


def stage_scan(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint32)
    out = np.empty_like(x)
    _check(lib().dance_stage_scan(_p(x, C.c_uint32), x.shape[0], _p(out, C.c_uint32)), "dance_stage_scan")
    return out


# ----------------------------------------------------------- stitched build

def stitched_row_cap(label_offsets: np.ndarray, label_points: np.ndarray, N: int, R_small: int,
                     R_stitched: int) -> int:
    """Row width that holds every label of a point: max labels per point x
    min(R_small, R_stitched)."""
    per = np.bincount(np.asarray(label_points, np.int64), minlength=N) if len(label_points) else np.zeros(1, int)
    return max(1, int(per.max()) * min(R_small, R_stitched))


def stitched_build(data: np.ndarray, label_offsets: np.ndarray, label_points: np.ndarray, R_small: int = 32,
                   L_small: int = 100, C_: int = 96, STEPS: int = 64, R_stitched: int = 64, row_cap: int | None = None):
    """dance_stitched_build: per-label standard builds over the label postings
    (label -> ascending point ids, CSR), remapped into one global graph on
    the device. Returns (graph N x row_cap, degree, label medoids, stats)."""
    data = np.ascontiguousarray(data)
    N, dim = data.shape
    off = np.ascontiguousarray(label_offsets, np.uint32)
    pts = np.ascontiguousarray(label_points, np.uint32)
    nl = off.shape[0] - 1
    cap = row_cap or stitched_row_cap(off, pts, N, R_small, R_stitched)
    graph = np.empty((N, cap), np.uint32)
    degree = np.empty(N, np.uint32)
    medoids = np.empty(max(1, nl), np.uint32)
    _check(lib().dance_stitched_build(data.ctypes.data, dtype_code(data), N, dim, _p(off, C.c_uint32),
                                      _p(pts, C.c_uint32), nl, R_small, L_small, C_, STEPS, R_stitched, cap,
                                      graph.ctypes.data, degree.ctypes.data, _p(medoids, C.c_uint32)),
           "dance_stitched_build")
    return graph, degree, medoids[:nl], last_stitched_stats()


def stitched_build_resident(d_data: int, dtype: int, N: int, dim: int, label_offsets: np.ndarray,
                            label_points: np.ndarray, R_small: int, L_small: int, C_: int, STEPS: int,
                            R_stitched: int, row_cap: int, d_graph: int, d_degree: int) -> np.ndarray:
    """dance_stitched_build_resident on device rows and outputs; returns the
    label medoids (host)."""
    off = np.ascontiguousarray(label_offsets, np.uint32)
    pts = np.ascontiguousarray(label_points, np.uint32)
    nl = off.shape[0] - 1
    medoids = np.empty(max(1, nl), np.uint32)
    _check(lib().dance_stitched_build_resident(d_data, dtype, N, dim, _p(off, C.c_uint32), _p(pts, C.c_uint32), nl,
                                               R_small, L_small, C_, STEPS, R_stitched, row_cap, d_graph, d_degree,
                                               _p(medoids, C.c_uint32)), "dance_stitched_build_resident")
    return medoids[:nl]


def last_stitched_stats() -> dict:
    s = DanceStitchedStats()
    lib().dance_get_last_stitched_stats(C.byref(s))
    return struct_dict(s)


# ------------------------------------------------------------- query search

def _opt_ptr(a):
    return None if a is None else a.ctypes.data


def search(data: np.ndarray, graph: np.ndarray, degree: np.ndarray, starts, queries: np.ndarray, k: int, L: int,
           label_offsets=None, labels=None, query_labels=None):
    """dance_search: best-first search of host queries over a built graph on
    host arrays. starts: int (shared entry point), one per query, or a list
    with one sequence of entry points per query (dance_search_multistart);
    the label arrays (all or none) restrict the search to points carrying the
    query's label. Returns (ids, dists), each nq x k."""
    data = np.ascontiguousarray(data)
    graph = np.ascontiguousarray(graph, np.uint32)
    degree = np.ascontiguousarray(degree, np.uint32)
    return _search(False, data.ctypes.data, dtype_code(data), data.shape[0], data.shape[1],
                   graph.ctypes.data, degree.ctypes.data, graph.shape[1], starts, queries, k, L, label_offsets,
                   labels, query_labels)


def search_resident(d_data: int, dtype: int, N: int, dim: int, d_graph: int, d_degree: int, R: int, starts,
                    queries: np.ndarray, k: int, L: int, label_offsets=None, labels=None, query_labels=None):
    """dance_search_resident: as search() with base rows, graph and degrees
    given as device pointers (e.g. torch data_ptr())."""
    return _search(True, d_data, dtype, N, dim, d_graph, d_degree, R, starts, queries, k, L,
                   label_offsets, labels, query_labels)


def start_lists(starts, nq: int):
    """A list of per-query start sequences -> (offsets nq + 1, flat ids);
    None for a single start or one start per query."""
    if not (isinstance(starts, (list, tuple)) and any(np.ndim(x) > 0 for x in starts)):
        return None
    lists = [np.atleast_1d(np.asarray(x, np.uint32)) for x in starts]
    if len(lists) != nq:
        raise ValueError(f"{len(lists)} start lists for {nq} queries")
    off = np.zeros(nq + 1, np.uint32)
    off[1:] = np.cumsum([x.shape[0] for x in lists])
    flat = np.concatenate(lists) if off[-1] else np.zeros(1, np.uint32)
    return off, np.ascontiguousarray(flat, np.uint32)


def _search(resident, data_p, dtype, N, dim, graph_p, degree_p, R, starts, queries, k, L, label_offsets, labels,
            query_labels):
    queries = np.ascontiguousarray(queries)
    nq = queries.shape[0]
    ids = np.empty((nq, k), np.uint32)
    dists = np.empty((nq, k), np.float32)
    opt = [None if a is None else np.ascontiguousarray(a, np.uint32) for a in (label_offsets, labels, query_labels)]
    ptrs = [_opt_ptr(a) for a in opt]
    multi = start_lists(starts, nq)
    if multi is None:
        st = np.atleast_1d(np.asarray(starts, np.uint32))
        fn = lib().dance_search_resident if resident else lib().dance_search
        rc = fn(data_p, dtype, N, dim, graph_p, degree_p, R, _p(st, C.c_uint32), st.shape[0], queries.ctypes.data,
                nq, k, L, *ptrs, _p(ids, C.c_uint32), _p(dists, C.c_float))
    else:
        off, flat = multi
        fn = lib().dance_search_multistart_resident if resident else lib().dance_search_multistart
        rc = fn(data_p, dtype, N, dim, graph_p, degree_p, R, _p(off, C.c_uint32), _p(flat, C.c_uint32),
                queries.ctypes.data, nq, k, L, *ptrs, _p(ids, C.c_uint32), _p(dists, C.c_float))
    _check(rc, "dance_search")
    return ids, dists


def last_search_stats() -> dict:
    s = DanceSearchStats()
    lib().dance_get_last_search_stats(C.byref(s))
    return struct_dict(s)


def recall_at_k(found: np.ndarray, gt: np.ndarray, k: int = 10) -> float:
    """Mean |found[:k] & gt[:k]| / k over queries (gt rows may hold INVALID
    padding when fewer than k points qualify; those slots are not counted)."""
    hits, total = 0, 0
    for f, g in zip(found, gt):
        g = [x for x in g[:k] if x != INVALID]
        total += len(g)
        hits += len(set(f[:k].tolist()) & set(g))
    return hits / max(1, total)


# ------------------------------------------------------------------ workloads

def synth_f32(seed: int, stream: int, n: int, dim: int, centers: int, sigma: float,
              normalize: bool = True) -> np.ndarray:
    out = np.empty((n, dim), dtype=np.float32)
    _check(lib().dance_synth_f32(seed, stream, n, dim, centers, sigma, int(normalize), _p(out, C.c_float)),
           "dance_synth_f32")
    return out


def synth_u8(seed: int, stream: int, n: int, dim: int, centers: int, sigma: float) -> np.ndarray:
    out = np.empty((n, dim), dtype=np.uint8)
    _check(lib().dance_synth_u8(seed, stream, n, dim, centers, sigma, _p(out, C.c_uint8)), "dance_synth_u8")
    return out


# The benchmark configurations (seeded synthetic generators: i.i.d. or
# Gaussian-mixture rows, L2-normalised for float); stream 0 = base vectors,
# stream 1 = queries.
CONFIGS = {
    "c1": dict(kind="f32", n=100_000, dim=96, centers=0, sigma=1.0, nq=1_000, R=64, L=100, C=80, STEPS=64),
    "c2": dict(kind="f32", n=1_000_000, dim=96, centers=256, sigma=0.3, nq=10_000, R=64, L=100, C=80, STEPS=64),
    "c3": dict(kind="f32", n=10_000_000, dim=96, centers=256, sigma=0.3, nq=10_000, R=64, L=100, C=80, STEPS=64),
    "c4": dict(kind="u8", n=10_000_000, dim=128, centers=1024, sigma=0.3, nq=10_000, R=64, L=100, C=80, STEPS=64),
}


def make_workload(cfg: dict, n: int | None = None, seed: int = 42):
    n = cfg["n"] if n is None else n
    if cfg["kind"] == "f32":
        base = synth_f32(seed, 0, n, cfg["dim"], cfg["centers"], cfg["sigma"], True)
        q = synth_f32(seed, 1, cfg["nq"], cfg["dim"], cfg["centers"], cfg["sigma"], True)
    else:
        base = synth_u8(seed, 0, n, cfg["dim"], cfg["centers"], cfg["sigma"])
        q = synth_u8(seed, 1, cfg["nq"], cfg["dim"], cfg["centers"], cfg["sigma"])
    return base, q
