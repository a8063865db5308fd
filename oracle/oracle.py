"""ctypes front-end of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module as the checker. Product code never imports it.

Parity status of each oracle function (how it is pinned; see tests/test_oracle.py):
  hash_u32, det_neighbor  pinned: bijectivity via the closed-form inverse of the
                          xorshift-multiply steps; range/bump properties.
  distance (f32/f16/u8)   pinned: u8 exact integer; f32/f16 within the fp32
                          error bound of an fp64 evaluation; symmetry; d(a,a)=0.
  medoid                  pinned: fp64 brute force of the same candidate/sample
                          scheme on small N.
  init_graph              pinned: closed form (hashed neighbours, distances).
  prune                   pinned: textbook RobustPrune (DiskANN Alg. 2 + fill)
                          restated independently in Python, plus invariants.
  reverse_merge           pinned: CSR == transpose of the first-R forward
                          entries with ascending sources; merge invariants and an
                          independent Python restatement.
  robust_insert           pinned: an independent Python restatement of the
                          occlude / victim / append / replace rule on tiny
                          integer rows with exact ties, full rows, invalid and
                          self members, FLT_MAX and NaN stored distances.
  search                  pinned: with a huge alpha nothing is occluded or
                          replaced, so the work row is the current row followed
                          by the expansion order, compared with an independent
                          best-first search (whole graph and beam eviction).
  vnew2_build             pinned as the composition of the pinned stages
                          (alpha schedule, coarse steps, final fill) and end to
                          end by recall@10 against exact brute force.
  v8_build                pinned: its own C-stride double-buffered composition
                          of the pinned stages equals vnew2_build without the
                          heavy cap, and differs from vnew2_build with the cap
                          where a reverse list exceeds the threshold.
  cpu_vamana_build        the recall gate's comparator and the timed CPU
                          baseline (DiskANN's algorithm restated; upstream
                          DiskANN is not available offline). Pinned against
                          independent Python statements of the paper's
                          RobustPrune with DiskANN's alpha ladder, of the
                          best-first search, and of the whole single-thread
                          build, on tie-heavy integer rows; a full-beam search
                          equals brute force (tests/test_cpu_vamana.py).
  merge_shards            pinned: mix64 by its closed-form inverse; the merge by
                          an independent Python restatement (sets, sorted())
                          on random shard sets, plus invariants; error codes
                          on malformed inputs (tests/test_merge_oracle.py).
  query_search            pinned: exact top-k on a complete graph; equal to the
                          independently written beam_search on integer data
                          (exact distances).
  filtered_random_graph   pinned: distinct non-self ids, degree min(16, R, N-1),
                          first entry = closed-form hash draw.
  filtered_prune          pinned: equals a greedy in (distance, id) order that
                          keeps a candidate iff no kept one occludes it, with
                          label coverage as Python set inclusion; with one
                          shared label it is textbook RobustPrune without fill.
  filtered_merge          pinned: ordered min-distance dedupe (Python dict) when
                          no quota applies; single-label rows keep the first
                          quota candidates carrying the label.
  filtered_build          pinned by the stages above plus build invariants
                          (no self / duplicate / invalid edge, degree <= R,
                          label-compatible edges) and recall on labelled
                          queries.
  filtered task / union   pinned: a restated canonical pool in Python (slot =
  searches                insertion order, eviction of the worst) with and
                          without eviction; multi-label quota by a brute-force
                          restatement with cardinality ties.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
INVALID = 0xFFFFFFFF
DTYPE = {np.dtype(np.float32): 0, np.dtype(np.uint8): 1, np.dtype(np.float16): 2}

_u32p = C.POINTER(C.c_uint32)
_f32p = C.POINTER(C.c_float)
_LIB = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        u32, f32, vp, i32, u64 = C.c_uint32, C.c_float, C.c_void_p, C.c_int, C.c_uint64
        L.oracle_hash_u32.argtypes = [u32]
        L.oracle_hash_u32.restype = u32
        L.oracle_det_neighbor.argtypes = [u32, u32, u32]
        L.oracle_det_neighbor.restype = u32
        L.oracle_half_round.argtypes = [C.c_double]
        L.oracle_half_round.restype = C.c_uint16
        L.oracle_half_sq_of_diff.argtypes = [C.c_uint16, C.c_uint16]
        L.oracle_half_sq_of_diff.restype = f32
        L.oracle_robust_insert.argtypes = [vp, i32, u32, u32, u32, u32, u32, f32, f32, _u32p, _f32p, _u32p]
        L.oracle_robust_insert.restype = None
        L.oracle_filtered_task_search.argtypes = [vp, i32, u32, u32, u32, _u32p, _u32p, u32, _u32p, u32, u32,
                                                  _u32p, _u32p, u32, u32, u32, u32, u32, _u32p, _f32p]
        L.oracle_filtered_task_search.restype = None
        L.oracle_filtered_ordinary_search.argtypes = [vp, i32, u32, u32, u32, _u32p, _u32p, u32, _u32p, u32,
                                                      _u32p, _u32p, u32, u32, u32, u32, u32, _u32p, _f32p]
        L.oracle_filtered_ordinary_search.restype = None
        L.oracle_distance.argtypes = [vp, i32, u32, u32, u32]
        L.oracle_distance.restype = f32
        L.oracle_distance_many.argtypes = [vp, i32, u32, _u32p, _u32p, u64, _f32p]
        L.oracle_distance_many.restype = None
        L.oracle_medoid.argtypes = [vp, i32, u32, u32, _f32p, _u32p]
        L.oracle_medoid.restype = u32
        L.oracle_init_graph.argtypes = [vp, i32, u32, u32, u32, u32, _u32p, _u32p, _u32p, _u32p, _f32p]
        L.oracle_init_graph.restype = None
        L.oracle_search.argtypes = [vp, i32, u32, u32, u32, u32, u32, u32, f32, u32, _u32p, _u32p, _u32p,
                                    _u32p, _f32p]
        L.oracle_search.restype = u64
        L.oracle_reverse_merge.argtypes = [vp, i32, u32, u32, u32, u32, _u32p, _u32p, _f32p, u32, u32,
                                           _u32p, _u32p]
        L.oracle_reverse_merge.restype = u64
        L.oracle_prune.argtypes = [vp, i32, u32, u32, u32, u32, u32, f32, _u32p, _u32p, _f32p, _u32p, _u32p]
        L.oracle_prune.restype = None
        L.oracle_vnew2_build.argtypes = [vp, i32, u32, u32, u32, u32, u32, u32, u32, f32, u32, u32, u32, _u32p,
                                         _u32p, _u32p]
        L.oracle_vnew2_build.restype = i32
        L.oracle_v8_build.argtypes = [vp, i32, u32, u32, u32, u32, u32, u32, u32, f32, u32, _u32p, _u32p, _u32p]
        L.oracle_v8_build.restype = i32
        L.oracle_cpu_vamana_build.argtypes = [vp, i32, u32, u32, u32, u32, f32, u32, i32, i32, _u32p, _u32p]
        L.oracle_cpu_vamana_build.restype = u32
        L.oracle_cpu_occlude.argtypes = [vp, i32, u32, _u32p, _f32p, u32, u32, f32, u32, _u32p]
        L.oracle_cpu_occlude.restype = u32
        L.oracle_cpu_greedy.argtypes = [vp, i32, u32, u32, _u32p, _u32p, u32, u32, vp, u32, u32, _u32p, _u32p]
        L.oracle_cpu_greedy.restype = u32
        L.oracle_beam_search.argtypes = [vp, i32, u32, u32, _u32p, _u32p, u32, u32, vp, u32, u32, u32, _u32p]
        L.oracle_beam_search.restype = u64
        L.oracle_bruteforce_knn.argtypes = [vp, i32, u32, u32, vp, u32, u32, _u32p, _f32p]
        L.oracle_bruteforce_knn.restype = None
        L.oracle_filtered_random_graph.argtypes = [u32, u32, u32, u32, _u32p, _u32p]
        L.oracle_filtered_random_graph.restype = None
        L.oracle_filtered_build.argtypes = [vp, i32, u32, u32, u32, u32, u32, u32, u32, f32, _u32p, _u32p, u32,
                                            _u32p, u32, u32, u32, u32, u32, _u32p, _u32p, C.POINTER(u64)]
        L.oracle_filtered_build.restype = i32
        L.oracle_filtered_round_log.argtypes = [C.POINTER(C.c_uint64)]
        L.oracle_filtered_round_log.restype = None
        L.oracle_filtered_prune.argtypes = [vp, i32, u32, u32, u32, f32, _u32p, _u32p, u32, _u32p, _f32p, u32,
                                            _u32p]
        L.oracle_filtered_prune.restype = u32
        L.oracle_filtered_merge.argtypes = [u32, u32, u32, u32, _u32p, _u32p, u32, u32, _u32p, _u32p, u32,
                                            _u32p, _f32p, _u32p, _f32p, u32, _u32p, _f32p]
        L.oracle_filtered_merge.restype = u32
        L.oracle_query_search.argtypes = [vp, i32, u32, u32, _u32p, _u32p, u32, _u32p, u32, _u32p, vp, u32, u32,
                                          u32, vp, vp, vp, _u32p, _f32p]
        L.oracle_query_search.restype = u64
        L.oracle_filtered_shortlist.argtypes = [u32, u32, _u32p, _u32p, u32, u32, u32, u32, _u32p, _f32p, u32,
                                                _u32p, _f32p]
        L.oracle_filtered_shortlist.restype = u32
        L.oracle_mix64.argtypes = [u64]
        L.oracle_mix64.restype = u64
        L.oracle_edge_hash.argtypes = [u32, u32, u64]
        L.oracle_edge_hash.restype = u32
        L.oracle_merge_shards.argtypes = [C.c_char_p] * 4 + [u64, u32] + [C.c_char_p] * 2 + [u64, C.POINTER(u64)]
        L.oracle_merge_shards.restype = i32
        L.oracle_partition_assign.argtypes = [vp, i32, u64, u32, C.POINTER(C.c_float), u32, u32, C.POINTER(u32)]
        L.oracle_partition_assign.restype = None
        L.oracle_num_threads.argtypes = []
        L.oracle_num_threads.restype = i32
        _LIB = L
    return _LIB


def _p(a, t=C.c_uint32):
    return a.ctypes.data_as(C.POINTER(t))


def _dt(data: np.ndarray) -> int:
    return DTYPE[data.dtype]


def hash_u32(x: int) -> int:
    return int(lib().oracle_hash_u32(x))


def det_neighbor(node: int, k: int, N: int) -> int:
    return int(lib().oracle_det_neighbor(node, k, N))


def half_round(x: float) -> int:
    """binary16 bits of x rounded to nearest even (the oracle's helper)."""
    return int(lib().oracle_half_round(float(x)))


def half_sq_of_diff(a_bits: int, b_bits: int) -> float:
    """binary16 (a - b)^2, widened (one element of the fp16 distance)."""
    return float(np.float32(lib().oracle_half_sq_of_diff(a_bits, b_bits)))


def distance(data: np.ndarray, a: int, b: int) -> float:
    data = np.ascontiguousarray(data)
    return float(np.float32(lib().oracle_distance(data.ctypes.data, _dt(data), data.shape[1], a, b)))


def distances(data: np.ndarray, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    data = np.ascontiguousarray(data)
    a = np.ascontiguousarray(a, np.uint32)
    b = np.ascontiguousarray(b, np.uint32)
    out = np.empty(a.shape[0], np.float32)
    lib().oracle_distance_many(data.ctypes.data, _dt(data), data.shape[1], _p(a), _p(b), a.shape[0],
                               _p(out, C.c_float))
    return out


def medoid(data: np.ndarray):
    data = np.ascontiguousarray(data)
    nc = min(1024, data.shape[0])
    scores = np.empty(nc, np.float32)
    cands = np.empty(nc, np.uint32)
    m = lib().oracle_medoid(data.ctypes.data, _dt(data), data.shape[0], data.shape[1], _p(scores, C.c_float),
                            _p(cands))
    return int(m), scores, cands


class State:
    """Graph state in the device layout: cur N x R, work/wd N x C."""

    def __init__(self, cur, deg_cur, work, deg_work, wd):
        self.cur, self.deg_cur, self.work, self.deg_work, self.wd = cur, deg_cur, work, deg_work, wd

    @staticmethod
    def empty(N, R, C_):
        return State(np.full((N, R), INVALID, np.uint32), np.zeros(N, np.uint32),
                     np.full((N, C_), INVALID, np.uint32), np.zeros(N, np.uint32),
                     np.full((N, C_), np.finfo(np.float32).max, np.float32))

    def copy(self):
        return State(self.cur.copy(), self.deg_cur.copy(), self.work.copy(), self.deg_work.copy(), self.wd.copy())

    def ptrs(self):
        return _p(self.cur), _p(self.deg_cur), _p(self.work), _p(self.deg_work), _p(self.wd, C.c_float)


def init_graph(data: np.ndarray, R: int, C_: int) -> State:
    data = np.ascontiguousarray(data)
    s = State.empty(data.shape[0], R, C_)
    lib().oracle_init_graph(data.ctypes.data, _dt(data), data.shape[0], data.shape[1], R, C_, *s.ptrs())
    return s


def search(data: np.ndarray, s: State, L: int, steps: int, alpha: float, start: int) -> State:
    data = np.ascontiguousarray(data)
    s = s.copy()
    N, R = s.cur.shape
    lib().oracle_search(data.ctypes.data, _dt(data), N, data.shape[1], R, L, s.work.shape[1], steps, alpha, start,
                        *s.ptrs())
    return s


def robust_insert(data: np.ndarray, node: int, x: int, d_px: float, alpha: float, row, drow, deg: int):
    """One online robust insert into a work row of capacity len(row); returns
    (row, drow, deg) after it."""
    row = np.ascontiguousarray(row, np.uint32).copy()
    drow = np.ascontiguousarray(drow, np.float32).copy()
    d = np.array([deg], np.uint32)
    lib().oracle_robust_insert(data.ctypes.data, _dt(data), data.shape[0], data.shape[1], row.shape[0], node, x,
                               d_px, alpha, _p(row), _p(drow, C.c_float), _p(d))
    return row, drow, int(d[0])


def reverse_merge(data: np.ndarray, s: State, heavy_threshold: int = 0, heavy_sample: int = 0):
    data = np.ascontiguousarray(data)
    s = s.copy()
    N, R = s.cur.shape
    off = np.zeros(N + 1, np.uint32)
    ids = np.zeros(N * R, np.uint32)
    n = lib().oracle_reverse_merge(data.ctypes.data, _dt(data), N, data.shape[1], R, s.work.shape[1],
                                   _p(s.work), _p(s.deg_work), _p(s.wd, C.c_float), heavy_threshold, heavy_sample,
                                   _p(off), _p(ids))
    return s, off, ids[:n]


def prune(data: np.ndarray, s: State, min_degree: int, alpha: float) -> State:
    data = np.ascontiguousarray(data)
    s = s.copy()
    N, R = s.cur.shape
    lib().oracle_prune(data.ctypes.data, _dt(data), N, data.shape[1], R, s.work.shape[1], min_degree, alpha,
                       _p(s.work), _p(s.deg_work), _p(s.wd, C.c_float), _p(s.cur), _p(s.deg_cur))
    return s


def vnew2_build(data: np.ndarray, R=64, L=100, C_=80, STEPS=64, iters=4, alpha=1.2, heavy_threshold=0,
                heavy_sample=0, alpha_from=None):
    """alpha_from: first iteration that prunes with alpha (default: the last,
    the reference's default schedule)."""
    data = np.ascontiguousarray(data)
    alpha_from = iters - 1 if alpha_from is None else alpha_from
    N = data.shape[0]
    graph = np.empty((N, R), np.uint32)
    deg = np.empty(N, np.uint32)
    med = np.zeros(1, np.uint32)
    rc = lib().oracle_vnew2_build(data.ctypes.data, _dt(data), N, data.shape[1], R, L, C_, STEPS, iters, alpha,
                                  alpha_from, heavy_threshold, heavy_sample, _p(graph), _p(deg), _p(med))
    if rc != 0:
        raise ValueError(f"oracle_vnew2_build rejected the parameters (rc={rc})")
    return graph, deg, int(med[0])


def v8_build(data: np.ndarray, R=64, L=100, C_=80, STEPS=64, iters=4, alpha=1.2, alpha_from=None):
    """The v8 builder (gpu_vamana_uint8.cu) with its C-stride double-buffered
    graphs and no reverse heavy cap; alpha_from as in vnew2_build."""
    data = np.ascontiguousarray(data)
    alpha_from = iters - 1 if alpha_from is None else alpha_from
    N = data.shape[0]
    graph = np.empty((N, R), np.uint32)
    deg = np.empty(N, np.uint32)
    med = np.zeros(1, np.uint32)
    rc = lib().oracle_v8_build(data.ctypes.data, _dt(data), N, data.shape[1], R, L, C_, STEPS, iters, alpha,
                               alpha_from, _p(graph), _p(deg), _p(med))
    if rc != 0:
        raise ValueError(f"oracle_v8_build rejected the parameters (rc={rc})")
    return graph, deg, int(med[0])


CPU_POOLS = {"diskann": 0, "paper": 1}


def cpu_vamana_build(data: np.ndarray, R=64, L=100, alpha=1.2, maxc=750, threads=0, pool="diskann"):
    """DiskANN-style CPU Vamana (cpu_baselines.cpp); threads=1 inserts in id
    order (deterministic), 0 uses every OpenMP thread. pool "diskann" prunes
    the expanded set of the search (DiskANN's search_for_point_and_prune),
    "paper" that set plus the point's current neighbours (Alg. 2 of the
    paper)."""
    data = np.ascontiguousarray(data)
    N = data.shape[0]
    graph = np.empty((N, R), np.uint32)
    deg = np.empty(N, np.uint32)
    start = lib().oracle_cpu_vamana_build(data.ctypes.data, _dt(data), N, data.shape[1], R, L, alpha, maxc,
                                          threads, CPU_POOLS[pool], _p(graph), _p(deg))
    return graph, deg, int(start)


def cpu_occlude(data: np.ndarray, ids, dists, R, alpha, maxc=750):
    """The CPU Vamana's RobustPrune alone: candidates sorted by (distance,
    id), cut to maxc, alpha ladder; returns the kept ids in selection order."""
    data = np.ascontiguousarray(data)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    dists = np.ascontiguousarray(dists, dtype=np.float32)
    out = np.empty(max(1, R), np.uint32)
    k = lib().oracle_cpu_occlude(data.ctypes.data, _dt(data), data.shape[1], _p(ids), dists.ctypes.data_as(_f32p),
                                 ids.shape[0], R, alpha, maxc, _p(out))
    return out[:k].tolist()


def cpu_greedy(data: np.ndarray, graph, degree, start, query: np.ndarray, L):
    """The CPU Vamana's greedy search alone from `start` for one query row:
    (expanded ids in expansion order, final beam ids)."""
    data = np.ascontiguousarray(data)
    graph = np.ascontiguousarray(graph, dtype=np.uint32)
    degree = np.ascontiguousarray(degree, dtype=np.uint32)
    q = np.ascontiguousarray(query.reshape(1, -1).astype(data.dtype))
    N, R = graph.shape
    exp = np.empty(N, np.uint32)
    beam = np.empty(L, np.uint32)
    k = lib().oracle_cpu_greedy(data.ctypes.data, _dt(data), N, data.shape[1], _p(graph), _p(degree), R, start,
                                q.ctypes.data, 0, L, _p(exp), _p(beam))
    return exp[:k].tolist(), [int(b) for b in beam if b != INVALID]


def beam_search(data, graph, degree, start, queries, k, L):
    data = np.ascontiguousarray(data)
    queries = np.ascontiguousarray(queries, dtype=data.dtype)
    graph = np.ascontiguousarray(graph, np.uint32)
    degree = np.ascontiguousarray(degree, np.uint32)
    out = np.empty((queries.shape[0], k), np.uint32)
    lib().oracle_beam_search(data.ctypes.data, _dt(data), data.shape[0], data.shape[1], _p(graph), _p(degree),
                             graph.shape[1], start, queries.ctypes.data, queries.shape[0], k, L, _p(out))
    return out


def bruteforce_knn(data, queries, k):
    data = np.ascontiguousarray(data)
    queries = np.ascontiguousarray(queries, dtype=data.dtype)
    ids = np.empty((queries.shape[0], k), np.uint32)
    d = np.empty((queries.shape[0], k), np.float32)
    lib().oracle_bruteforce_knn(data.ctypes.data, _dt(data), data.shape[0], data.shape[1], queries.ctypes.data,
                                queries.shape[0], k, _p(ids), _p(d, C.c_float))
    return ids, d


def recall_at_k(found: np.ndarray, gt: np.ndarray, k: int = 10) -> float:
    hits = 0
    for f, g in zip(found[:, :k], gt[:, :k]):
        hits += len(set(f.tolist()) & set(g.tolist()))
    return hits / (gt.shape[0] * k)


def num_threads() -> int:
    return int(lib().oracle_num_threads())


# ------------------------------------------------------------ filtered build

def filtered_random_graph(N: int, R: int, initial_degree: int = 16, seed: int = 42):
    g = np.empty((N, R), np.uint32)
    d = np.empty(N, np.uint32)
    lib().oracle_filtered_random_graph(N, R, initial_degree, seed, _p(g), _p(d))
    return g, d


def filtered_build(data: np.ndarray, offsets: np.ndarray, labels: np.ndarray, starts: np.ndarray,
                   num_labels: int, R: int = 64, L: int = 100, filtered_L: int = 100, C_: int = 750,
                   STEPS: int = 64, alpha: float = 1.2, universal: int = INVALID, global_start: int = INVALID,
                   rounds: int = 3, publish_R: int = 0):
    """canonical_v2 filtered build. Float32 rows are searched as fp16 (the
    reference converts float input, src/gpu_vamana_filtered.cu:6497-6503).
    With 0 < publish_R < R the publish step prunes the graph to publish_R
    (the graph then has publish_R columns). Returns (rc, graph, degree, diag[12])."""
    if data.dtype == np.float32:
        data = data.astype(np.float16)
    data = np.ascontiguousarray(data)
    N, dim = data.shape
    g = np.empty((N, R), np.uint32)
    d = np.empty(N, np.uint32)
    diag = np.zeros(12, np.uint64)
    offsets = np.ascontiguousarray(offsets, np.uint32)
    labels = np.ascontiguousarray(labels, np.uint32)
    starts = np.ascontiguousarray(starts, np.uint32)
    rc = lib().oracle_filtered_build(data.ctypes.data, _dt(data), N, dim, R, L, filtered_L, C_, STEPS, alpha,
                                     _p(offsets), _p(labels), int(labels.shape[0]), _p(starts), num_labels,
                                     universal, global_start, rounds, publish_R, _p(g), _p(d),
                                     diag.ctypes.data_as(C.POINTER(C.c_uint64)))
    if 0 < publish_R < R:
        g = np.ascontiguousarray(g.ravel()[:N * publish_R].reshape(N, publish_R))
    return rc, g, d, diag


def filtered_round_log() -> np.ndarray:
    """Per round of the last filtered_build (rows x [changed, touched,
    reverse proposals]; 3 rows, zero beyond its rounds)."""
    out = np.zeros(9, np.uint64)
    lib().oracle_filtered_round_log(out.ctypes.data_as(C.POINTER(C.c_uint64)))
    return out.reshape(3, 3)


def filtered_prune(data: np.ndarray, offsets: np.ndarray, labels: np.ndarray, row: int, ids: np.ndarray,
                   ds: np.ndarray, R: int, alpha: float) -> np.ndarray:
    data = np.ascontiguousarray(data)
    ids = np.ascontiguousarray(ids, np.uint32)
    ds = np.ascontiguousarray(ds, np.float32)
    out = np.empty(R, np.uint32)
    n = lib().oracle_filtered_prune(data.ctypes.data, _dt(data), data.shape[0], data.shape[1], R, alpha,
                                    _p(np.ascontiguousarray(offsets, np.uint32)),
                                    _p(np.ascontiguousarray(labels, np.uint32)), row, _p(ids), _p(ds, C.c_float),
                                    ids.shape[0], _p(out))
    return out[:n]


def _search_inputs(data, offsets, labels, starts, graph, degree):
    return (np.ascontiguousarray(data), np.ascontiguousarray(offsets, np.uint32),
            np.ascontiguousarray(labels, np.uint32), np.ascontiguousarray(starts, np.uint32),
            np.ascontiguousarray(graph, np.uint32), np.ascontiguousarray(degree, np.uint32))


def filtered_task_search(data, offsets, labels, starts, num_labels: int, universal: int, graph, degree, row: int,
                         label: int, pool_cap: int, keep: int, steps: int):
    """One per-label task search (the oracle's canonical_filtered_task_search);
    returns the `keep` emitted (ids, distances)."""
    data, offsets, labels, starts, graph, degree = _search_inputs(data, offsets, labels, starts, graph, degree)
    ids = np.empty(keep, np.uint32)
    d = np.empty(keep, np.float32)
    lib().oracle_filtered_task_search(data.ctypes.data, _dt(data), data.shape[0], data.shape[1], graph.shape[1],
                                      _p(offsets), _p(labels), labels.shape[0], _p(starts), num_labels, universal,
                                      _p(graph), _p(degree), row, label, pool_cap, keep, steps, _p(ids),
                                      _p(d, C.c_float))
    return ids, d


def filtered_ordinary_search(data, offsets, labels, starts, num_labels: int, graph, degree, row: int,
                             pool_cap: int, keep: int, steps: int, global_start: int):
    """One union (ordinary) search (the oracle's canonical_ordinary_search)."""
    data, offsets, labels, starts, graph, degree = _search_inputs(data, offsets, labels, starts, graph, degree)
    ids = np.empty(keep, np.uint32)
    d = np.empty(keep, np.float32)
    lib().oracle_filtered_ordinary_search(data.ctypes.data, _dt(data), data.shape[0], data.shape[1],
                                          graph.shape[1], _p(offsets), _p(labels), labels.shape[0], _p(starts),
                                          num_labels, _p(graph), _p(degree), row, pool_cap, keep, steps,
                                          global_start, _p(ids), _p(d, C.c_float))
    return ids, d


def filtered_merge(N: int, R: int, C_: int, keep: int, offsets, labels, num_labels: int, graph, degree, row: int,
                   task_ids, task_d, ord_ids, ord_d):
    offsets = np.ascontiguousarray(offsets, np.uint32)
    labels = np.ascontiguousarray(labels, np.uint32)
    graph = np.ascontiguousarray(graph, np.uint32)
    degree = np.ascontiguousarray(degree, np.uint32)
    task_ids = np.ascontiguousarray(task_ids, np.uint32)
    task_d = np.ascontiguousarray(task_d, np.float32)
    ord_ids = np.ascontiguousarray(ord_ids, np.uint32)
    ord_d = np.ascontiguousarray(ord_d, np.float32)
    out_i = np.empty(C_, np.uint32)
    out_d = np.empty(C_, np.float32)
    n = lib().oracle_filtered_merge(N, R, C_, keep, _p(offsets), _p(labels), int(labels.shape[0]), num_labels,
                                    _p(graph), _p(degree), row, _p(task_ids), _p(task_d, C.c_float),
                                    _p(ord_ids), _p(ord_d, C.c_float), ord_ids.shape[0], _p(out_i),
                                    _p(out_d, C.c_float))
    return out_i[:n], out_d[:n]


def start_csr(starts, nq):
    """starts as one id, one id per query, or one sequence of ids per query
    -> (offsets or None, flat starts)."""
    if isinstance(starts, (list, tuple)) and any(np.ndim(s) > 0 for s in starts):
        lists = [np.atleast_1d(np.asarray(s, np.uint32)) for s in starts]
        if len(lists) != nq:
            raise ValueError("one start list per query")
        off = np.zeros(nq + 1, np.uint32)
        off[1:] = np.cumsum([x.shape[0] for x in lists])
        flat = np.concatenate(lists) if lists else np.zeros(0, np.uint32)
        return off, np.ascontiguousarray(flat if flat.size else np.zeros(1, np.uint32))
    return None, np.atleast_1d(np.asarray(starts, np.uint32))


def query_search(data, graph, degree, starts, queries, k, L, label_offsets=None, labels=None, query_labels=None):
    """Canonical-distance best-first search (DiskANN search semantics);
    starts: one id, one per query, or a list of start lists (one per query);
    returns (ids, dists, distance count)."""
    data = np.ascontiguousarray(data)
    queries = np.ascontiguousarray(queries)
    graph = np.ascontiguousarray(graph, np.uint32)
    degree = np.ascontiguousarray(degree, np.uint32)
    nq = queries.shape[0]
    soff, starts = start_csr(starts, nq)
    ids = np.empty((nq, k), np.uint32)
    dd = np.empty((nq, k), np.float32)
    opt = [None if a is None else np.ascontiguousarray(a, np.uint32) for a in (label_offsets, labels, query_labels)]
    ptrs = [None if a is None else a.ctypes.data for a in opt]
    n = lib().oracle_query_search(data.ctypes.data, _dt(data), data.shape[0], data.shape[1], _p(graph), _p(degree),
                                  graph.shape[1], _p(starts), starts.shape[0], None if soff is None else _p(soff),
                                  queries.ctypes.data, nq, k, L, *ptrs, _p(ids), _p(dd, C.c_float))
    return ids, dd, int(n)


MERGE_DEFAULT_SEED = 0x9E3779B97F4A7C15


def mix64(x: int) -> int:
    return int(lib().oracle_mix64(x))


def edge_hash(src: int, dst: int, seed: int = MERGE_DEFAULT_SEED) -> int:
    return int(lib().oracle_edge_hash(src, dst, seed))


def merge_shards(vamana_prefix: str, vamana_suffix: str, idmaps_prefix: str, idmaps_suffix: str, nshards: int,
                 max_degree: int, output_vamana: str, medoids_file: str, seed: int = MERGE_DEFAULT_SEED):
    """CPU restatement of diskann::merge_shards_gpu; returns (rc, {self_loops, unique_edges, output_edges})."""
    cnt = (C.c_uint64 * 3)()
    rc = lib().oracle_merge_shards(vamana_prefix.encode(), vamana_suffix.encode(), idmaps_prefix.encode(),
                                   idmaps_suffix.encode(), nshards, max_degree, output_vamana.encode(),
                                   medoids_file.encode(), seed, cnt)
    return int(rc), {"self_loops": int(cnt[0]), "unique_edges": int(cnt[1]), "output_edges": int(cnt[2])}


def filtered_shortlist(offsets, labels, num_labels: int, universal: int, R: int, row: int, ids, ds):
    """One rare-label shortlist (the publish step's candidate choice); returns (ids, dists)."""
    offsets = np.ascontiguousarray(offsets, np.uint32)
    labels = np.ascontiguousarray(labels, np.uint32)
    ids = np.ascontiguousarray(ids, np.uint32)
    ds = np.ascontiguousarray(ds, np.float32)
    oi = np.empty(max(R, 1), np.uint32)
    od = np.empty(max(R, 1), np.float32)
    n = lib().oracle_filtered_shortlist(offsets.shape[0] - 1, R, _p(offsets), _p(labels), int(labels.shape[0]),
                                        num_labels, universal, row, _p(ids), _p(ds, C.c_float), int(ids.shape[0]),
                                        _p(oi), _p(od, C.c_float))
    return oi[:n], od[:n]


def partition_assign(data: np.ndarray, centers: np.ndarray, k_base: int) -> np.ndarray:
    """Each row's k_base nearest centers (fp64 squared L2 in dimension order,
    ties to the lower center); returns N x k_base uint32."""
    data = np.ascontiguousarray(data)
    centers = np.ascontiguousarray(centers, np.float32)
    out = np.empty((data.shape[0], k_base), np.uint32)
    lib().oracle_partition_assign(data.ctypes.data, 0 if data.dtype == np.float32 else 1, data.shape[0],
                                  data.shape[1], _p(centers, C.c_float), centers.shape[0], k_base, _p(out))
    return out
