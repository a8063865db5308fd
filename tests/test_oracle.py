"""Pins the CPU oracle (CPU only; no GPU).

Each oracle function is checked against something it does not share code
with: closed-form inverses, fp64 evaluations with error bounds, brute force on
tiny inputs, and independent textbook restatements written here in Python.
"""
import numpy as np
import pytest

from oracle import oracle as O

INV = 0xFFFFFFFF
FMAX = np.finfo(np.float32).max
M32 = 0xFFFFFFFF


# ---------------------------------------------------------------- hashes

def _unxorshift(x, s):
    # inverse of x ^= x >> s on 32 bits
    y = x
    for _ in range(32 // s + 1):
        y = x ^ (y >> s)
    return y & M32


def _inverse_hash(h):
    # vnew2.cu:169-177 is xorshift16, *0x7feb352d, xorshift15, *0x846ca68b,
    # xorshift16; undo each step in reverse order.
    x = _unxorshift(h, 16)
    x = (x * pow(0x846CA68B, -1, 1 << 32)) & M32
    x = _unxorshift(x, 15)
    x = (x * pow(0x7FEB352D, -1, 1 << 32)) & M32
    return _unxorshift(x, 16)


def test_hash_is_the_documented_bijection():
    rng = np.random.default_rng(0)
    xs = [0, 1, 2, 0xFFFFFFFF, 0x80000000] + rng.integers(0, 1 << 32, 2000, dtype=np.uint64).tolist()
    for x in xs:
        assert _inverse_hash(O.hash_u32(int(x))) == int(x)
    assert O.hash_u32(0) == 0
    # distinct inputs -> distinct outputs (spot check of injectivity)
    hs = {O.hash_u32(i) for i in range(20000)}
    assert len(hs) == 20000


@pytest.mark.parametrize("N", [2, 3, 7, 1000, 100_003])
def test_det_neighbor_range_and_bump(N):
    for node in list(range(min(N, 50))) + [N - 1]:
        for k in list(range(70)) + [1024, 1031]:
            v = O.det_neighbor(node, k, N)
            assert 0 <= v < N and v != node
            h = O.hash_u32((node * 0x9E3779B1 + k * 0x85EBCA6B + 17) & M32) % N
            assert v == (h if h != node else (h + 1) % N)
    assert O.det_neighbor(0, 0, 1) == INV


# ---------------------------------------------------------------- distances

@pytest.mark.parametrize("dim", [1, 7, 96, 100, 128, 333])
def test_distance_f32_within_fp32_bound(dim):
    rng = np.random.default_rng(dim)
    x = rng.standard_normal((64, dim)).astype(np.float32)
    a = rng.integers(0, 64, 500)
    b = rng.integers(0, 64, 500)
    got = O.distances(x, a, b).astype(np.float64)
    exact = ((x[a].astype(np.float64) - x[b].astype(np.float64)) ** 2).sum(1)
    # |fl(sum) - sum| <= (dim + 2) u sum for a sum of non-negative terms
    bound = (dim + 3) * 2.0 ** -24 * exact + 1e-30
    assert np.all(np.abs(got - exact) <= bound)
    # symmetry (bitwise) and zero self-distance
    assert np.array_equal(O.distances(x, a, b).view(np.uint32), O.distances(x, b, a).view(np.uint32))
    assert np.all(O.distances(x, a, a) == 0.0)


@pytest.mark.parametrize("dim", [1, 33, 128, 192])
def test_distance_u8_exact(dim):
    rng = np.random.default_rng(dim)
    x = rng.integers(0, 256, (50, dim), dtype=np.uint8)
    a = rng.integers(0, 50, 300)
    b = rng.integers(0, 50, 300)
    exact = ((x[a].astype(np.int64) - x[b].astype(np.int64)) ** 2).sum(1)
    assert np.array_equal(O.distances(x, a, b), exact.astype(np.float32))
    # extreme values
    y = np.zeros((2, dim), np.uint8)
    y[1] = 255
    assert O.distance(y, 0, 1) == float(dim * 255 * 255)


def _np_half_sq(a16, b16):
    """__hmul2(__hsub2(a, b), same) with numpy binary16 arithmetic, widened.
    numpy evaluates float16 operations in float32 and rounds once to float16;
    float32 carries 24 >= 2*11 + 2 bits, so that double rounding equals the
    single binary16 rounding of the exact result."""
    with np.errstate(over="ignore", invalid="ignore"):
        t = (a16 - b16).astype(np.float16)
        return (t * t).astype(np.float16).astype(np.float32)


def test_half_round_matches_numpy():
    rng = np.random.default_rng(11)
    xs = np.concatenate([
        rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
        # ties at every binade and in the subnormal range, overflow boundary
        (np.arange(1, 2048, dtype=np.float64) + 0.5) * 2.0 ** -24,
        (1024 + np.arange(0, 1024) + 0.5) * 2.0 ** rng.integers(-24, 6, 1024),
        [65504.0, 65519.99, 65520.0, 65536.0, 1e300, 2.0 ** -25, 2.0 ** -25 * 1.0001, 3 * 2.0 ** -26,
         0.0, -0.0, np.inf, -np.inf],
    ])
    xs = np.concatenate([xs, -xs])
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([O.half_round(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want), xs[got != want][:5]
    assert O.half_round(float("nan")) & 0x7C00 == 0x7C00 and O.half_round(float("nan")) & 0x3FF


def test_half_sq_of_diff_matches_numpy_binary16():
    rng = np.random.default_rng(12)
    a = (rng.standard_normal(30000) * 10.0 ** rng.integers(-6, 3, 30000)).astype(np.float16)
    b = (rng.standard_normal(30000) * 10.0 ** rng.integers(-6, 3, 30000)).astype(np.float16)
    # |a-b| above 256: the binary16 square overflows to inf (the widened fp32
    # form would stay finite); subnormal differences; equal values
    a = np.concatenate([a, np.float16([300.0, -200.0, 1.0, 6e-5, 0.5, 65504.0])])
    b = np.concatenate([b, np.float16([0.0, 100.0, 1.0, 5.9e-5, 0.5 + 2 ** -11, -65504.0])])
    want = _np_half_sq(a, b)
    got = np.array([O.half_sq_of_diff(int(x), int(y)) for x, y in zip(a.view(np.uint16), b.view(np.uint16))],
                   np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.isinf(got[-6]) and np.isinf(got[-5]) and np.isinf(got[-1])


def test_distance_f16_small_dims_exact():
    """dim 2: one pair, (float(sq0) + float(sq1)) exactly. dim 1: the odd
    tail alone, widened first and squared in fp32."""
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((200, 2)) * 4).astype(np.float16)
    a = rng.integers(0, 200, 500)
    b = rng.integers(0, 200, 500)
    sq = _np_half_sq(x[a], x[b])
    want = sq[:, 0] + sq[:, 1]
    assert np.array_equal(O.distances(x, a, b).view(np.uint32), want.view(np.uint32))
    x1 = np.ascontiguousarray(x[:, :1])
    t = x1[a, 0].astype(np.float32) - x1[b, 0].astype(np.float32)
    assert np.array_equal(O.distances(x1, a, b).view(np.uint32), (t * t).view(np.uint32))


@pytest.mark.parametrize("dim", [8, 50, 96, 97, 33])
def test_distance_f16_binary16_terms(dim):
    """The fp16 distance sums the binary16 per-element squares (plus an fp32
    square for an odd dim's last element): within the fp32 summation bound of
    the fp64 sum of those terms, and far from the widened form where the
    binary16 rounding of a difference moves it."""
    rng = np.random.default_rng(dim)
    x = rng.standard_normal((40, dim)).astype(np.float16)
    a = rng.integers(0, 40, 200)
    b = rng.integers(0, 40, 200)
    got = O.distances(x, a, b).astype(np.float64)
    terms = _np_half_sq(x[a], x[b]).astype(np.float64)
    if dim % 2:
        t = x[a, -1].astype(np.float64) - x[b, -1].astype(np.float64)
        terms[:, -1] = t * t
    exact = terms.sum(1)
    assert np.all(np.abs(got - exact) <= (dim + 3) * 2.0 ** -24 * exact + 1e-30)
    # symmetric bitwise, zero self-distance
    assert np.array_equal(O.distances(x, a, b).view(np.uint32), O.distances(x, b, a).view(np.uint32))
    assert np.all(O.distances(x, a, a) == 0.0)
    # a row pair whose binary16 difference overflows its square: inf, where
    # the widened form would give a finite value
    y = np.zeros((2, dim), np.float16)
    y[0, 0], y[1, 0] = 300.0, 0.0
    assert np.isinf(O.distance(y, 0, 1))
    if dim % 2:
        # the odd tail is squared in fp32: finite
        z = np.zeros((2, dim), np.float16)
        z[0, -1] = 300.0
        assert O.distance(z, 0, 1) == 90000.0


# ---------------------------------------------------------------- medoid

def test_medoid_matches_fp64_bruteforce():
    rng = np.random.default_rng(5)
    N, dim = 600, 24
    x = rng.standard_normal((N, dim)).astype(np.float32)
    m, scores, cands = O.medoid(x)
    nc, ns = min(1024, N), min(4096, N)
    want_c = np.array([O.hash_u32((w * 9973 + 17) & M32) % N for w in range(nc)])
    assert np.array_equal(cands, want_c)
    samples = np.array([O.hash_u32((s * 10007 + 131) & M32) % N for s in range(ns)])
    x64 = x.astype(np.float64)
    ref = np.array([((x64[samples[samples != c]] - x64[c]) ** 2).sum() / ns for c in want_c])
    assert np.allclose(scores, ref, rtol=1e-5)
    best = ref.min()
    assert ref[list(want_c).index(m)] <= best * (1 + 1e-5)


# ---------------------------------------------------------------- init

def test_init_graph_closed_form():
    rng = np.random.default_rng(2)
    N, dim, R, C = 300, 16, 12, 20
    x = rng.standard_normal((N, dim)).astype(np.float32)
    s = O.init_graph(x, R, C)
    for v in range(N):
        nb = [O.det_neighbor(v, k, N) for k in range(R)]
        assert s.cur[v].tolist() == nb
        assert s.work[v, :R].tolist() == nb and np.all(s.work[v, R:] == INV)
        assert np.array_equal(s.wd[v, :R], O.distances(x, np.full(R, v), np.array(nb)))
        assert np.all(s.wd[v, R:] == FMAX)
    assert np.all(s.deg_cur == R) and np.all(s.deg_work == R)


# ---------------------------------------------------------------- prune

def random_work_state(x, R, C, seed):
    rng = np.random.default_rng(seed)
    N = x.shape[0]
    s = O.State.empty(N, R, C)
    ids = rng.integers(0, N, (N, C)).astype(np.uint32)
    ids[rng.random((N, C)) < 0.08] = INV
    selfm = rng.random((N, C)) < 0.03
    ids[selfm] = np.broadcast_to(np.arange(N, dtype=np.uint32)[:, None], (N, C))[selfm]
    dupm = rng.random((N, C - 1)) < 0.08
    ids[:, 1:][dupm] = ids[:, :-1][dupm]
    a = np.repeat(np.arange(N, dtype=np.uint32), C)
    b = ids.ravel()
    ok = b < N
    d = np.full(N * C, FMAX, np.float32)
    d[ok] = O.distances(x, a[ok], b[ok])
    d = d.reshape(N, C)
    d[rng.random((N, C)) < 0.02] = FMAX
    s.work, s.wd = ids, d
    s.deg_work = rng.integers(0, C + 1, N).astype(np.uint32)
    return s


def textbook_prune(x, node, ids, ds, R, alpha, min_degree):
    """RobustPrune (DiskANN Alg. 2) over the candidate slots, selection by
    (distance, slot); then the nearest-first fill of unused ids."""
    N = x.shape[0]
    V = [(float(d), i, int(v)) for i, (v, d) in enumerate(zip(ids, ds))
         if v != INV and v < N and v != node and np.float32(d) < FMAX]
    out = []
    while V:
        p = min(V)
        out.append((p[2], p[0]))
        if len(out) == R:
            break
        rest = []
        for (d, i, v) in V:
            if v == p[2]:
                continue
            dpv = O.distance(x, p[2], v)
            if p[0] <= d and np.float32(alpha) * np.float32(dpv) <= np.float32(d):
                continue
            rest.append((d, i, v))
        V = rest
    chosen = {v for v, _ in out}
    fill = sorted((float(d), i, int(v)) for i, (v, d) in enumerate(zip(ids, ds))
                  if v != INV and v < N and v != node and np.float32(d) < FMAX)
    for d, i, v in fill:
        if len(out) >= min(min_degree, R):
            break
        if v in chosen:
            continue
        chosen.add(v)
        out.append((v, d))
    return out


@pytest.mark.parametrize("alpha,min_degree", [(1.0, 0), (1.2, 0), (1.2, 16), (1.5, 64)])
def test_prune_matches_textbook(alpha, min_degree):
    rng = np.random.default_rng(9)
    N, dim, R, C = 200, 12, 16, 40
    x = rng.standard_normal((N, dim)).astype(np.float32)
    s0 = random_work_state(x, R, C, seed=4)
    s = O.prune(x, s0, min_degree, alpha)
    for v in range(N):
        deg = min(int(s0.deg_work[v]), C)
        want = textbook_prune(x, v, s0.work[v, :deg], s0.wd[v, :deg], R, alpha, min_degree)
        k = int(s.deg_cur[v])
        assert [int(i) for i in s.cur[v, :k]] == [w for w, _ in want]
        assert np.all(s.cur[v, k:] == INV)
        assert np.array_equal(s.wd[v, :k], np.array([d for _, d in want], np.float32))
        assert s.deg_work[v] == k


def test_prune_invariants():
    rng = np.random.default_rng(1)
    N, dim, R, C, alpha = 300, 16, 24, 60, 1.2
    x = rng.standard_normal((N, dim)).astype(np.float32)
    s0 = random_work_state(x, R, C, seed=8)
    s = O.prune(x, s0, 0, alpha)
    for v in range(N):
        k = int(s.deg_cur[v])
        out = [int(i) for i in s.cur[v, :k]]
        assert len(set(out)) == k and v not in out and all(i < N for i in out)
        d = s.wd[v, :k]
        assert np.all(np.diff(d) >= 0)  # selection order is nearest first
        for i in range(k):  # no selected node occludes a later one
            for j in range(i + 1, k):
                assert alpha * O.distance(x, out[i], out[j]) > d[j]


# ---------------------------------------------------------------- reverse

def test_reverse_csr_is_transpose_with_ascending_sources():
    rng = np.random.default_rng(3)
    N, dim, R, C = 400, 8, 10, 24
    x = rng.standard_normal((N, dim)).astype(np.float32)
    s0 = random_work_state(x, R, C, seed=5)
    _, off, ids = O.reverse_merge(x, s0)
    want = {}
    for src in range(N):
        for i in range(min(int(s0.deg_work[src]), R)):
            t = int(s0.work[src, i])
            if t != INV and t < N and t != src:
                want.setdefault(t, []).append(src)
    for t in range(N):
        seg = ids[off[t]:off[t + 1]].tolist()
        assert seg == sorted(want.get(t, []))


def textbook_merge(x, t, row, drow, deg, srcs, C):
    row, drow = list(row), list(drow)
    for s in srcs:
        if s == t or s in row[:deg]:
            continue
        d = O.distance(x, t, s)
        if deg < C:
            row[deg], drow[deg] = s, d
            deg += 1
            continue
        w = int(np.argmax(np.array(drow, np.float32)))  # first index of the max
        if np.float32(d) < np.float32(drow[w]):
            row[w], drow[w] = s, d
    return row, drow, deg


def test_reverse_merge_matches_textbook():
    rng = np.random.default_rng(6)
    N, dim, R, C = 300, 8, 12, 20
    x = rng.standard_normal((N, dim)).astype(np.float32)
    s0 = random_work_state(x, R, C, seed=7)
    s, off, ids = O.reverse_merge(x, s0)
    for t in range(N):
        row, drow, deg = textbook_merge(x, t, s0.work[t].tolist(), s0.wd[t].tolist(),
                                        min(int(s0.deg_work[t]), C), ids[off[t]:off[t + 1]].tolist(), C)
        assert s.work[t].tolist() == row
        assert np.array_equal(s.wd[t], np.array(drow, np.float32))
        assert int(s.deg_work[t]) == deg


# ---------------------------------------------------------------- search

def test_search_invariants():
    rng = np.random.default_rng(11)
    N, dim, R, L, C = 800, 16, 16, 40, 32
    x = rng.standard_normal((N, dim)).astype(np.float32)
    s0 = O.init_graph(x, R, C)
    m, _, _ = O.medoid(x)
    s = O.search(x, s0, L, 24, 1.0, m)
    for v in range(N):
        k = int(s.deg_work[v])
        assert k <= C
        row = [int(i) for i in s.work[v, :k] if i != INV]
        assert v not in row
        # The hashed init may repeat a neighbour; the work row starts as a copy
        # of the current row, and the online insert never adds a duplicate.
        cur = [int(i) for i in s0.cur[v]]
        for i in set(row):
            assert row.count(i) == 1 or row.count(i) <= cur.count(i)
        assert np.array_equal(s.wd[v, :k][s.work[v, :k] != INV],
                              O.distances(x, np.full(len(row), v), np.array(row, np.uint32)))
        assert np.all(s.work[v, k:] == INV)


def test_build_recall_and_cpu_vamana():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((3000, 32)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    q = rng.standard_normal((200, 32)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    gt, _ = O.bruteforce_knn(x, q, 10)
    g, deg, m = O.vnew2_build(x, 24, 48, 32, 32)
    assert np.all(deg <= 24) and m < 3000
    r1 = O.recall_at_k(O.beam_search(x, g, deg, m, q, 10, 64), gt)
    g2, deg2, st = O.cpu_vamana_build(x, 24, 48, 1.2)
    r2 = O.recall_at_k(O.beam_search(x, g2, deg2, st, q, 10, 64), gt)
    assert r1 > 0.9 and r2 > 0.9


def test_bruteforce_knn_exact():
    rng = np.random.default_rng(13)
    x = rng.standard_normal((500, 10)).astype(np.float32)
    q = rng.standard_normal((20, 10)).astype(np.float32)
    ids, d = O.bruteforce_knn(x, q, 5)
    full = ((q[:, None, :].astype(np.float64) - x[None].astype(np.float64)) ** 2).sum(2)
    assert np.array_equal(ids, np.argsort(full, axis=1, kind="stable")[:, :5])


def test_build_rejects_bad_parameters():
    x = np.zeros((10, 4), np.float32)
    with pytest.raises(ValueError):
        O.vnew2_build(x, 8, 10, 4, 4)  # C < R
    with pytest.raises(ValueError):
        O.vnew2_build(x, 0, 10, 8, 4)


# ------------------------------------------------- online robust insert

def restated_robust_insert(x, node, cand, d_px, alpha, row, drow, deg):
    """The online insert of vnew2.cu:759-877, restated from the reference
    source with Python lists: skip an invalid / self / present candidate;
    drop it when a row member y with d_py <= d_px has alpha * d(y, x) <= d_px;
    else overwrite the farthest member it alpha-dominates (d_py > d_px and
    alpha * d(x, y) <= d_py; first slot on ties), else append while the row
    has room, else overwrite the farthest member (first slot on ties) when
    closer than it."""
    N, C = x.shape[0], len(row)
    row, drow = list(row), [np.float32(v) for v in drow]
    deg = min(deg, C)
    a, dpx = np.float32(alpha), np.float32(d_px)
    if cand >= N or cand == node or cand in row[:deg]:
        return row, drow, deg
    members = [i for i in range(deg) if row[i] < N and row[i] != node]
    for i in members:
        if drow[i] <= dpx and a * np.float32(O.distance(x, row[i], cand)) <= dpx:
            return row, drow, deg
    finite = [i for i in members if drow[i] == drow[i]]
    worst = None
    if finite:
        top = max(drow[i] for i in finite)
        worst = min(i for i in finite if drow[i] == top)
    dominated = [i for i in members if drow[i] > dpx and a * np.float32(O.distance(x, cand, row[i])) <= drow[i]]
    if dominated:
        top = max(drow[i] for i in dominated)
        v = min(i for i in dominated if drow[i] == top)
        row[v], drow[v] = cand, dpx
    elif deg < C:
        row[deg], drow[deg] = cand, dpx
        deg += 1
    elif worst is not None and dpx < drow[worst]:
        row[worst], drow[worst] = cand, dpx
    return row, drow, deg


@pytest.mark.parametrize("seed", range(6))
def test_robust_insert_matches_restatement(seed):
    """Tiny rows of small-integer vectors, so exact ties are common: d_py ==
    d_px, alpha * d == d_px (alpha 0.5 / 1 / 2 are exact), full rows,
    invalid and self members, FLT_MAX and NaN stored distances, present,
    invalid and self candidates."""
    rng = np.random.default_rng(100 + seed)
    N, dim = 24, 3
    x = rng.integers(0, 3, (N, dim)).astype(np.uint8)
    for trial in range(1500):
        C = int(rng.integers(1, 7))
        node = int(rng.integers(0, N))
        row = rng.integers(0, N, C).astype(np.uint32)
        row[rng.random(C) < 0.15] = INV
        row[rng.random(C) < 0.1] = node
        drow = np.array([O.distance(x, node, int(v)) if v < N else FMAX for v in row], np.float32)
        drow[rng.random(C) < 0.1] = FMAX
        drow[rng.random(C) < 0.05] = np.nan
        deg = int(rng.integers(0, C + 1))
        cand = int(rng.integers(0, N)) if rng.random() > 0.05 else INV
        if rng.random() < 0.1 and deg:
            cand = int(row[rng.integers(0, deg)])
        d_px = O.distance(x, node, cand) if cand < N else FMAX
        if rng.random() < 0.2 and deg:  # tie a stored distance
            d_px = float(drow[rng.integers(0, deg)])
        alpha = float(rng.choice([0.5, 1.0, 1.2, 2.0]))
        got = O.robust_insert(x, node, cand, d_px, alpha, row, drow, deg)
        want = restated_robust_insert(x, node, cand, d_px, alpha, row.tolist(), drow.tolist(), deg)
        assert got[0].tolist() == want[0], (trial, node, cand, d_px, alpha, row, drow, deg)
        assert np.array_equal(got[1].view(np.uint32), np.array(want[1], np.float32).view(np.uint32))
        assert got[2] == want[2]


# ------------------------------------------------- search (pool + steps)

def textbook_best_first(x, node, cur, deg_cur, wd_row, start, L, steps):
    """Best-first search with a beam of the L nearest candidates (DiskANN
    Alg. 1; no slot layout): seeds are the start, the node's own neighbours at
    their stored distances and the 8 hashed seeds h(node, 1024 + k); each step
    expands the nearest unexpanded candidate, at most min(steps, L) steps.
    Returns the expansion order. Valid for inputs with distinct distances."""
    N = x.shape[0]
    pool = {}

    def offer(v, d):
        if v >= N or v == node or v in pool:
            return
        if len(pool) < L:
            pool[v] = [np.float32(d), False]
            return
        far = max(pool, key=lambda u: pool[u][0])
        if np.float32(d) < pool[far][0]:
            del pool[far]
            pool[v] = [np.float32(d), False]

    if start < N and start != node:
        offer(start, O.distance(x, node, start))
    for i in range(int(deg_cur[node])):
        offer(int(cur[node, i]), wd_row[i])
    for k in range(8):
        s = O.det_neighbor(node, 1024 + k, N)
        if s < N:
            offer(s, O.distance(x, node, s))
    order = []
    for _ in range(min(steps, L)):
        open_ = [u for u in pool if not pool[u][1]]
        if not open_:
            break
        u = min(open_, key=lambda v: pool[v][0])
        pool[u][1] = True
        order.append(u)
        for j in range(int(deg_cur[u])):
            v = int(cur[u, j])
            if v < N and v != node:
                offer(v, O.distance(x, node, v))
    return order


@pytest.mark.parametrize("N,R,L,steps", [(60, 4, 80, 100), (120, 6, 24, 40), (200, 5, 16, 8), (90, 3, 10, 64),
                                         (150, 8, 60, 20)])
def test_search_expansion_order_matches_best_first(N, R, L, steps):
    """With alpha huge nothing is occluded or replaced, so the online insert
    appends every expanded node the row does not hold: the work row after the
    search is the current row followed by the expansion order. Compared with
    an independent best-first search, on random graphs (L >= N - 1: whole
    graph explored; L < N: beam eviction; steps below and above L)."""
    rng = np.random.default_rng(N * 7 + L)
    x = rng.standard_normal((N, 12)).astype(np.float32)
    C = R + min(steps, L) + 1
    s0 = O.State.empty(N, R, C)
    s0.cur = rng.integers(0, N, (N, R)).astype(np.uint32)
    s0.cur[rng.random((N, R)) < 0.05] = INV
    s0.deg_cur = rng.integers(1, R + 1, N).astype(np.uint32)
    for v in range(N):
        s0.cur[v, s0.deg_cur[v]:] = INV
        for i in range(int(s0.deg_cur[v])):
            u = int(s0.cur[v, i])
            s0.wd[v, i] = O.distance(x, v, u) if u < N and u != v else FMAX
    start = int(rng.integers(0, N))
    s = O.search(x, s0, L, steps, 1e30, start)
    for v in range(N):
        order = textbook_best_first(x, v, s0.cur, s0.deg_cur, s0.wd[v], start, L, steps)
        row = [int(u) if (u < N and u != v) else INV for u in s0.cur[v, :s0.deg_cur[v]]]
        for u in order:
            if u not in row:
                row.append(u)
        k = int(s.deg_work[v])
        assert k == len(row), v
        assert s.work[v, :k].tolist() == row, v


@pytest.mark.parametrize("iters,alpha_from", [(4, 0), (4, 1), (4, 2), (4, 3), (1, 0), (2, 1), (5, 4), (5, 0),
                                              (6, 5), (6, 0)])
def test_alpha_schedule_composes_the_stages(iters, alpha_from):
    """The reference's schedule knobs composed from the separately pinned
    stages: VAMANA_ITERS iterations (gpu_vamana_config.h:78-79, the loop at
    vnew2.cu:2517-2637), alpha from iteration VAMANA_ALPHA_FINAL_FROM_ITER on
    and 1 before (vnew2.cu:201-213; USE_ALPHA_FROM_FIRST_ITER is from = 0).
    Medoid, init, then per iteration search (steps capped at 64 in the first
    two), reverse merge and prune (fill to 64 in the last). From = iters - 1
    is the default schedule, and with alpha 1 the knob changes nothing."""
    rng = np.random.default_rng(30 + 7 * iters + alpha_from)
    x = rng.standard_normal((300, 16)).astype(np.float32)
    R, L, C_, steps, alpha = 12, 32, 24, 80, 1.2
    start, _, _ = O.medoid(x)
    s = O.init_graph(x, R, C_)
    for it in range(iters):
        a = alpha if it >= alpha_from else 1.0
        s = O.search(x, s, L, min(steps, L, 64) if it < 2 else min(steps, L), a, start)
        s, _, _ = O.reverse_merge(x, s)
        s = O.prune(x, s, 64 if it == iters - 1 else 0, a)
    g, d, m = O.vnew2_build(x, R, L, C_, steps, iters, alpha, alpha_from=alpha_from)
    assert m == start and np.array_equal(d, s.deg_cur) and np.array_equal(g, s.cur)
    if alpha_from == iters - 1:
        g0, d0, _ = O.vnew2_build(x, R, L, C_, steps, iters, alpha)
        assert np.array_equal(g, g0) and np.array_equal(d, d0)
    g1, d1, _ = O.vnew2_build(x, R, L, C_, steps, iters, 1.0, alpha_from=alpha_from)
    g2, d2, _ = O.vnew2_build(x, R, L, C_, steps, iters, 1.0)
    assert np.array_equal(g1, g2) and np.array_equal(d1, d2)


def test_more_iterations_change_the_graph():
    """The iteration count is live: one more search / merge / prune pass over
    the same rows gives another graph (a build that ignored the count would
    pass the composition test only at the default)."""
    x = np.random.default_rng(5).standard_normal((400, 16)).astype(np.float32)
    g4, d4, _ = O.vnew2_build(x, 12, 32, 24, 32, 4)
    g5, d5, _ = O.vnew2_build(x, 12, 32, 24, 32, 5)
    assert not (np.array_equal(g4, g5) and np.array_equal(d4, d5))
