"""Label-filtered GPU Vamana build: Python side of include/gpu_vamana_filtered.h.

Mirrors the reference's filtered builder interface
(/root/reference/include/gpu_vamana_filtered.h:79-123) and the host glue
DiskANN runs before calling it (label CSR canonicalisation, label entry
points, global start; reference integrations/dance-diskann-78256bba.patch:20245-20540).
All graph work runs in libdance_hip.so; this module marshals arrays.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import (DTYPE_F16, DTYPE_F32, DTYPE_U8, INVALID, DanceFilteredProfile, GPUFilteredVamanaStats, _check,
               _p, dtype_code, lib, struct_dict)

# Defaults of the reference's release path and of DiskANN's build parameters.
ROUNDS = 3
DISKANN_MAXC = 750


@dataclass
class LabelSet:
    """Per-point label lists in CSR form, sorted ascending without repeats."""
    offsets: np.ndarray  # N+1 uint32
    labels: np.ndarray   # total uint32
    num_labels: int

    @property
    def n(self) -> int:
        return self.offsets.shape[0] - 1

    def row(self, i: int) -> np.ndarray:
        return self.labels[self.offsets[i]:self.offsets[i + 1]]

    def postings(self) -> tuple[np.ndarray, np.ndarray]:
        """label -> points CSR (points ascending), labels >= num_labels skipped."""
        rows = np.repeat(np.arange(self.n, dtype=np.uint32), np.diff(self.offsets).astype(np.int64))
        keep = self.labels < self.num_labels
        lab, rows = self.labels[keep], rows[keep]
        order = np.argsort(lab, kind="stable")
        counts = np.bincount(lab, minlength=self.num_labels)
        off = np.zeros(self.num_labels + 1, np.uint32)
        off[1:] = np.cumsum(counts)
        return off, rows[order].astype(np.uint32)


def canonical_labels(rows: list, num_labels: int | None = None) -> LabelSet:
    """Sorted-unique label CSR from per-point label lists (reference
    patch:20269-20286 canonicalises DiskANN's label lists the same way)."""
    offs = np.zeros(len(rows) + 1, np.uint32)
    flat = []
    for i, r in enumerate(rows):
        u = sorted(set(int(x) for x in r))
        flat.extend(u)
        offs[i + 1] = offs[i] + len(u)
    labels = np.asarray(flat, np.uint32)
    nl = num_labels if num_labels is not None else (int(labels.max()) + 1 if labels.size else 0)
    return LabelSet(offs, labels, nl)


def synth_labels(n: int, vocab: int, min_per: int = 1, max_per: int = 8, zipf_s: float = 1.0,
                 seed: int = 42) -> LabelSet:
    """Seeded multi-label workload: a uniform count in [min_per, max_per] per
    point, that many distinct labels drawn Zipf(zipf_s) over `vocab` ids
    (rank r has weight 1/(r+1)^s) without replacement within a point."""
    if max_per > vocab:
        raise ValueError("max_per exceeds the vocabulary")
    rng = np.random.default_rng(seed)
    w = 1.0 / np.power(np.arange(1, vocab + 1, dtype=np.float64), zipf_s)
    cdf = np.cumsum(w / w.sum())
    want = rng.integers(min_per, max_per + 1, n).astype(np.int64)
    keys = np.empty(0, np.int64)
    have = np.zeros(n, np.int64)
    while True:
        short = np.nonzero(have < want)[0]
        if short.size == 0:
            break
        need = want[short] - have[short]
        rows = np.repeat(short, need)
        draws = np.minimum(np.searchsorted(cdf, rng.random(rows.size), side="right"), vocab - 1)
        # each short row draws its deficit; repeats collapse and are redrawn
        keys = np.unique(np.concatenate([keys, rows * vocab + draws]))
        have = np.bincount(keys // vocab, minlength=n)
    offs = np.zeros(n + 1, np.uint32)
    offs[1:] = np.cumsum(have)
    return LabelSet(offs, (keys % vocab).astype(np.uint32), vocab)


def zipf_labels(count: int, vocab: int, zipf_s: float = 1.0, seed: int = 43) -> np.ndarray:
    """One label per query, Zipf(zipf_s) over vocab ids."""
    rng = np.random.default_rng(seed)
    w = 1.0 / np.power(np.arange(1, vocab + 1, dtype=np.float64), zipf_s)
    cdf = np.cumsum(w / w.sum())
    return np.minimum(np.searchsorted(cdf, rng.random(count), side="right"), vocab - 1).astype(np.uint32)


START_CANDS = 25  # carriers drawn per label by the load-balanced rule


def _splitmix64(state: int) -> tuple[int, int]:
    state = (state + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
    return state, z ^ (z >> 31)


def balanced_label_starts(ls: LabelSet, universal: int = INVALID, seed: int = 1) -> np.ndarray:
    """Entry point per label by Filtered-DiskANN's load-balanced FindMedoid,
    the rule upstream DiskANN's Index::build_filtered_index applies right
    before the reference's GPU branch (patch:20239, consumed at :20288-20296):
    per label in ascending id order, START_CANDS carriers drawn uniformly with
    replacement, the first drawn of those that start the fewest labels so far
    wins and its count rises by one. Carriers of `universal` carry every label.
    Draws are splitmix64 outputs modulo the carrier count from `seed`, the
    stream build_memory_index uses (DISKANN_GPU_FILTERED_LABEL_START_SEED,
    default 1). INVALID for labels without carriers."""
    off, pts = ls.postings()
    nl = ls.num_labels
    uni = pts[off[universal]:off[universal + 1]] if universal < nl else np.empty(0, pts.dtype)
    starts = np.full(max(1, nl), INVALID, np.uint32)
    load = {}
    state = seed & 0xFFFFFFFFFFFFFFFF
    for l in range(nl):
        carriers = np.union1d(pts[off[l]:off[l + 1]], uni) if uni.size else pts[off[l]:off[l + 1]]
        if carriers.size == 0:
            continue
        best, best_load = None, None
        for _ in range(START_CANDS):
            state, r = _splitmix64(state)
            c = int(carriers[r % carriers.size])
            if best_load is None or load.get(c, 0) < best_load:
                best, best_load = c, load.get(c, 0)
        starts[l] = best
        load[best] = best_load + 1
    return starts


def start_hash(point: np.ndarray, label: int) -> np.ndarray:
    """The reference's hash of a (point, label) pair for extra search starts
    (integrations/dance-diskann-78256bba.patch:19836-19844): x = point << 32
    ^ label ^ 0x9e3779b97f4a7c15, the splitmix64 finaliser, low 32 bits."""
    with np.errstate(over="ignore"):
        x = (np.asarray(point, np.uint64) << np.uint64(32)) ^ np.uint64(label) ^ np.uint64(0x9E3779B97F4A7C15)
        x ^= x >> np.uint64(30)
        x *= np.uint64(0xBF58476D1CE4E5B9)
        x ^= x >> np.uint64(27)
        x *= np.uint64(0x94D049BB133111EB)
        x ^= x >> np.uint64(31)
    return (x & np.uint64(0xFFFFFFFF)).astype(np.uint32)


def extra_label_starts(ls: LabelSet, starts: np.ndarray, per_label: int) -> list:
    """Extra search starts per label, as the reference's filtered search picks
    them under DISKANN_FILTERED_SEARCH_EXTRA_STARTS=per_label (at most 16;
    patch:19817-19873): the label's carriers other than its start, the
    per_label smallest by (start_hash, point), in that order. One array per
    label (empty for labels without a start)."""
    per_label = min(int(per_label), 16)
    off, pts = ls.postings()
    out = []
    for l in range(ls.num_labels):
        c = pts[off[l]:off[l + 1]]
        if per_label <= 0 or l >= len(starts) or starts[l] == INVALID or c.size == 0:
            out.append(np.zeros(0, np.uint32))
            continue
        c = c[c != starts[l]]
        h = start_hash(c, l)
        order = np.lexsort((c, h))[:per_label]
        out.append(c[order].astype(np.uint32))
    return out


def query_starts(data: np.ndarray, queries: np.ndarray, qlabels: np.ndarray, starts: np.ndarray, extra: list,
                 select: int = 0) -> list:
    """Entry points of each query's filtered search (patch:20583-20625): the
    label's start and its extra starts, or with select > 0 only the select
    extra starts nearest to the query (DISKANN_FILTERED_SEARCH_EXTRA_START_SELECT,
    squared L2, ties to the smaller id), sorted and deduplicated."""
    out = []
    for r, l in enumerate(qlabels):
        ids = [int(starts[l])] if starts[l] != INVALID else []
        ex = extra[l]
        if select > 0 and ex.size:
            diff = data[ex].astype(np.float64) - queries[r].astype(np.float64)
            d = (diff * diff).sum(1)
            ex = ex[np.lexsort((ex, d))[:select]]
        out.append(sorted(set(ids) | set(int(v) for v in ex)))
    return out


def label_starts(data: np.ndarray, ls: LabelSet) -> np.ndarray:
    """Entry point per label: the point of the label nearest (squared L2, fp64)
    to the label's centroid; INVALID for labels without points (the
    build_memory_index option DANCE_LABEL_STARTS=centroid; its default is
    balanced_label_starts). Any in-label point is a valid entry for the
    builder."""
    off, pts = ls.postings()
    starts = np.full(max(1, ls.num_labels), INVALID, np.uint32)
    lab_of = np.repeat(np.arange(ls.num_labels), np.diff(off).astype(np.int64))
    if pts.size == 0:
        return starts
    dim = data.shape[1]
    cnt = np.diff(off).astype(np.float64)
    # per-dimension label sums (fp64; exact for integer rows)
    sums = np.empty((ls.num_labels, dim))
    for j in range(dim):
        sums[:, j] = np.bincount(lab_of, weights=data[pts, j].astype(np.float64), minlength=ls.num_labels)
    cent = sums / np.maximum(cnt, 1)[:, None]
    d = np.empty(pts.size)
    step = 1 << 18
    for s0 in range(0, pts.size, step):
        seg = slice(s0, s0 + step)
        d[seg] = ((data[pts[seg]].astype(np.float64) - cent[lab_of[seg]]) ** 2).sum(1)
    for l in np.nonzero(cnt)[0]:
        seg = slice(off[l], off[l + 1])
        j = int(np.argmin(d[seg]))
        starts[l] = pts[off[l] + j]
    return starts


def global_start(data: np.ndarray) -> int:
    """Point nearest to the centroid (DiskANN calculate_entry_point analogue)."""
    n = data.shape[0]
    mean = np.zeros(data.shape[1])
    step = 1 << 18
    for s0 in range(0, n, step):
        mean += data[s0:s0 + step].astype(np.float64).sum(0)
    mean /= max(1, n)
    d = np.empty(n)
    for s0 in range(0, n, step):
        d[s0:s0 + step] = ((data[s0:s0 + step].astype(np.float64) - mean) ** 2).sum(1)
    return int(np.argmin(d))


@dataclass
class FilteredResult:
    graph: np.ndarray   # N x R uint32, INVALID-padded rows
    degree: np.ndarray  # N uint32
    stats: dict
    profile: dict


def last_stats() -> dict:
    s = GPUFilteredVamanaStats()
    lib().gpu_vamana_filtered_get_last_stats(C.byref(s))
    return struct_dict(s)


def last_profile() -> dict:
    p = DanceFilteredProfile()
    lib().dance_get_last_filtered_profile(C.byref(p))
    return struct_dict(p)


def build_rc(data, ls: LabelSet, starts, R: int, L: int, filtered_L: int, C_: int = DISKANN_MAXC,
             STEPS: int = 64, alpha: float = 1.2, universal: int = INVALID, gstart: int = INVALID,
             rounds: int = ROUNDS, graph=None, degree=None, total: int | None = None) -> int:
    """Calls the C ABI and returns its code (no exception). data: uint8 /
    float32 host rows (reference entry points) or float16 (extension entry,
    rows searched as given); rounds != 3 also uses the extension entry."""
    N = ls.n if data is None else data.shape[0]
    dim = 0 if data is None else data.shape[1]
    graph = np.empty((N, R), np.uint32) if graph is None else graph
    degree = np.empty(N, np.uint32) if degree is None else degree
    starts = np.ascontiguousarray(starts, np.uint32)
    total = int(ls.labels.shape[0]) if total is None else total
    dptr = None if data is None else data.ctypes.data
    lab_args = (_p(ls.offsets, C.c_uint32), _p(ls.labels, C.c_uint32), total, _p(starts, C.c_uint32),
                ls.num_labels, universal, gstart)
    L_ = lib()
    code = DTYPE_U8 if data is None else dtype_code(data)
    if rounds == ROUNDS and code in (DTYPE_U8, DTYPE_F32):
        fn = L_.gpu_vamana_filtered_build_uint8 if code == DTYPE_U8 else L_.gpu_vamana_filtered_build_float
        return fn(dptr, N, dim, R, L, filtered_L, C_, STEPS, alpha, *lab_args, None, None, 0,
                  _p(graph, C.c_uint32), _p(degree, C.c_uint32))
    return L_.dance_filtered_build(dptr, code, N, dim, R, L, filtered_L, C_, STEPS, alpha, *lab_args, rounds,
                                   _p(graph, C.c_uint32), _p(degree, C.c_uint32))


def filtered_build(data: np.ndarray, ls: LabelSet, starts: np.ndarray | None = None, R: int = 64, L: int = 100,
                   filtered_L: int = 100, C_: int = DISKANN_MAXC, STEPS: int = 64, alpha: float = 1.2,
                   universal: int = INVALID, gstart: int | None = None, rounds: int = ROUNDS) -> FilteredResult:
    """gpu_vamana_filtered_build_{uint8,float} on host rows. With
    DISKANN_GPU_FILTERED_PUBLISH_DEGREE set to PR in (0, R) the graph has PR
    columns (the publish step)."""
    data = np.ascontiguousarray(data)
    if data.ndim != 2 or data.shape[0] != ls.n:
        raise ValueError("data must be N x dim with one label row per point")
    starts = label_starts(data, ls) if starts is None else starts
    gstart = global_start(data) if gstart is None else gstart
    graph = np.empty((data.shape[0], R), np.uint32)
    degree = np.empty(data.shape[0], np.uint32)
    _check(build_rc(data, ls, starts, R, L, filtered_L, C_, STEPS, alpha, universal, gstart, rounds, graph,
                    degree), "gpu_vamana_filtered_build")
    prof = last_profile()
    PR = int(prof["publish_degree"])  # below R after the publish step (DISKANN_GPU_FILTERED_PUBLISH_DEGREE)
    if PR < R:
        graph = np.ascontiguousarray(graph.ravel()[:data.shape[0] * PR].reshape(data.shape[0], PR))
    return FilteredResult(graph, degree, last_stats(), prof)


def filtered_build_resident(d_data: int, dtype: int, N: int, dim: int, ls: LabelSet, starts: np.ndarray, R: int,
                            L: int, filtered_L: int, C_: int, STEPS: int, alpha: float, universal: int,
                            gstart: int, d_graph: int, d_degree: int) -> None:
    """dance_filtered_build_resident on device pointers (torch data_ptr())."""
    starts = np.ascontiguousarray(starts, np.uint32)
    _check(lib().dance_filtered_build_resident(
        d_data, dtype, N, dim, R, L, filtered_L, C_, STEPS, alpha, _p(ls.offsets, C.c_uint32),
        _p(ls.labels, C.c_uint32), int(ls.labels.shape[0]), _p(starts, C.c_uint32), ls.num_labels, universal,
        gstart, d_graph, d_degree), "dance_filtered_build_resident")


__all__ = ["LabelSet", "canonical_labels", "synth_labels", "zipf_labels", "label_starts", "balanced_label_starts",
           "extra_label_starts", "query_starts", "start_hash", "global_start", "FilteredResult", "filtered_build", "filtered_build_resident", "build_rc", "last_stats", "last_profile", "ROUNDS",
           "DISKANN_MAXC", "DTYPE_F16", "DTYPE_F32", "DTYPE_U8"]
