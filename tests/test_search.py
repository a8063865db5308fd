"""Query search (dance_search): the CPU oracle is pinned by closed forms, the
GPU kernel must return the oracle's ids and canonical distances bit for bit,
unfiltered and with a label filter."""
import numpy as np
import pytest

import dance_amd as D
from dance_amd import INVALID
from dance_amd import filtered as F
from oracle import oracle as O


def test_oracle_search_on_complete_graph_is_exact_topk():
    """Every node links to all others: after the start's expansion the list
    holds the L nearest points, so the k best are the exact k nearest."""
    rng = np.random.default_rng(1)
    n, k = 200, 10
    x = rng.integers(0, 256, (n, 16), dtype=np.uint8)
    q = rng.integers(0, 256, (20, 16), dtype=np.uint8)
    g = np.array([[j for j in range(n) if j != i] + [INVALID] for i in range(n)], np.uint32)
    deg = np.full(n, n - 1, np.uint32)
    ids, dd, _ = O.query_search(x, g, deg, 0, q, k, 32)
    exact = ((q[:, None, :].astype(np.int64) - x[None].astype(np.int64)) ** 2).sum(-1)
    for r in range(20):
        order = np.lexsort((np.arange(n), exact[r]))[:k]
        assert ids[r].tolist() == order.tolist()
        assert np.array_equal(dd[r], exact[r][order].astype(np.float32))


def test_oracle_search_matches_reference_style_beam_search():
    """On integer data every distance is exact, so the canonical search equals
    the independently written sorted-beam search of the CPU baselines."""
    rng = np.random.default_rng(2)
    x = rng.integers(0, 256, (2000, 32), dtype=np.uint8)
    q = rng.integers(0, 256, (50, 32), dtype=np.uint8)
    g, d, med = O.vnew2_build(x, 24, 48, 40, 24)
    for L in (10, 40, 100):
        ids, _, _ = O.query_search(x, g, d, med, q, 10, L)
        want = O.beam_search(x, g, d, med, q, 10, L)
        assert np.array_equal(ids, want)


def test_oracle_multistart_pins():
    """Several entry points per query (DiskANN's init_ids): a one-entry list
    equals the single-start search; duplicates and ids >= N are ignored; the
    order of a list does not matter; every node as a start with L >= N gives
    the exact top-k; an empty list returns nothing."""
    rng = np.random.default_rng(8)
    n = 600
    x = rng.integers(0, 256, (n, 16), dtype=np.uint8)
    q = rng.integers(0, 256, (12, 16), dtype=np.uint8)
    g, d, med = O.vnew2_build(x, 16, 32, 24, 16)
    one = [[int(s)] for s in rng.integers(0, n, 12)]
    a, ad, _ = O.query_search(x, g, d, one, q, 10, 40)
    b, bd, _ = O.query_search(x, g, d, np.array([o[0] for o in one], np.uint32), q, 10, 40)
    assert np.array_equal(a, b) and np.array_equal(ad, bd)
    lists = [list(rng.integers(0, n, int(rng.integers(1, 70)))) for _ in range(12)]
    noisy = [l + l[:3] + [n, n + 5, INVALID] for l in lists]
    perm = [list(rng.permutation(l)) for l in lists]
    r0, _, _ = O.query_search(x, g, d, lists, q, 10, 40)
    for other in (noisy, perm):
        r1, _, _ = O.query_search(x, g, d, other, q, 10, 40)
        assert np.array_equal(r0, r1)
    full, fd, _ = O.query_search(x, g, d, [list(range(n))] * 12, q, 10, n)
    exact = ((q[:, None, :].astype(np.int64) - x[None].astype(np.int64)) ** 2).sum(-1)
    for r in range(12):
        assert full[r].tolist() == np.lexsort((np.arange(n), exact[r]))[:10].tolist()
    empty, ed, _ = O.query_search(x, g, d, [[]] * 12, q, 10, 40)
    assert np.all(empty == INVALID) and np.all(ed == np.finfo(np.float32).max)


def test_oracle_search_wide_list_on_complete_graph():
    """L = 1000 (the reference's widest published search list) on a complete
    graph of 1200 points: exact top-k."""
    rng = np.random.default_rng(11)
    n = 1200
    x = rng.integers(0, 256, (n, 8), dtype=np.uint8)
    q = rng.integers(0, 256, (5, 8), dtype=np.uint8)
    g = np.array([[j for j in range(n) if j != i] for i in range(n)], np.uint32)
    deg = np.full(n, n - 1, np.uint32)
    ids, _, _ = O.query_search(x, g, deg, 0, q, 64, 1000)
    exact = ((q[:, None, :].astype(np.int64) - x[None].astype(np.int64)) ** 2).sum(-1)
    for r in range(5):
        assert ids[r].tolist() == np.lexsort((np.arange(n), exact[r]))[:64].tolist()


def test_search_parameter_errors():
    x = np.zeros((10, 4), np.float32)
    g = np.zeros((10, 4), np.uint32)
    deg = np.zeros(10, np.uint32)
    for k, L in [(0, 10), (65, 100), (10, 5), (10, 1025)]:
        with pytest.raises(D.BuildError):
            D.search(x, g, deg, 0, x[:2], k, L)
    with pytest.raises(D.BuildError):  # partial label filter
        D.search(x, g, deg, 0, x[:2], 4, 8, label_offsets=np.zeros(11, np.uint32))
    with pytest.raises(ValueError):  # one start list per query
        D.search(x, g, deg, [[0], [1], [2]], x[:2], 4, 8)
    lib = D.lib()
    u32p = D.C.POINTER(D.C.c_uint32)
    ids = np.zeros((2, 4), np.uint32)
    dd = np.zeros((2, 4), np.float32)
    bad_off = np.array([0, 2, 1], np.uint32)  # decreasing offsets: rejected before any device call
    st = np.zeros(2, np.uint32)
    assert lib.dance_search_multistart(x.ctypes.data, 0, 10, 4, g.ctypes.data, deg.ctypes.data, 4,
                                       bad_off.ctypes.data_as(u32p), st.ctypes.data_as(u32p), x.ctypes.data, 2, 4,
                                       8, None, None, None, ids.ctypes.data_as(u32p),
                                       dd.ctypes.data_as(D.C.POINTER(D.C.c_float))) == -1


def make(kind, n, dim, seed):
    rng = np.random.default_rng(seed)
    if kind == "u8":
        return rng.integers(0, 256, (n, dim), dtype=np.uint8), rng.integers(0, 256, (200, dim), dtype=np.uint8)
    x = rng.standard_normal((n + 200, dim)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    if kind == "f16":
        x = x.astype(np.float16)
    return x[:n], x[n:]


@pytest.mark.gpu
@pytest.mark.parametrize("kind,dim", [("u8", 64), ("f32", 96), ("f16", 96), ("f32", 20)])
@pytest.mark.parametrize("L", [10, 64, 100, 200, 300, 500, 650, 1000])
def test_gpu_search_matches_oracle(kind, dim, L):
    x, q = make(kind, 3000, dim, seed=dim + L)
    g, d, med = O.vnew2_build(x, 32, 64, 48, 32)
    ids, dd = D.search(x, g, d, med, q, 10, L)
    oi, od, n = O.query_search(x, g, d, med, q, 10, L)
    assert np.array_equal(ids, oi)
    assert np.array_equal(dd.view(np.uint32), od.view(np.uint32))
    st = D.last_search_stats()
    # the forgetful visited cache may recompute a distance, never skip one
    assert st["capped_queries"] == 0 and st["distances"] >= n


@pytest.mark.gpu
def test_gpu_filtered_search_matches_oracle():
    x, q = make("u8", 3000, 64, seed=4)
    ls = F.synth_labels(3000, 20, 1, 3, 1.0, seed=5)
    starts = F.label_starts(x, ls)
    res = F.filtered_build(x, ls, starts, 32, 64, 64, 750, 32)
    rng = np.random.default_rng(6)
    ql = rng.integers(0, 20, q.shape[0]).astype(np.uint32)
    qs = starts[ql]
    ids, dd = D.search(x, res.graph, res.degree, qs, q, 10, 64, ls.offsets, ls.labels, ql)
    oi, od, _ = O.query_search(x, res.graph, res.degree, qs, q, 10, 64, ls.offsets, ls.labels, ql)
    assert np.array_equal(ids, oi) and np.array_equal(dd.view(np.uint32), od.view(np.uint32))
    for r in range(q.shape[0]):  # every result carries the query label
        for v in ids[r]:
            if v != INVALID:
                assert ql[r] in ls.row(int(v))


@pytest.mark.gpu
@pytest.mark.parametrize("L,filtered", [(40, False), (100, True), (1000, True), (300, False)])
def test_gpu_multistart_search_matches_oracle(L, filtered):
    """Several entry points per query: lists of 0..150 starts (more than one
    64-wide batch) with repeats and ids >= N, with and without the label
    filter; ids and distances bit-exact with the oracle."""
    x, q = make("u8", 3000, 64, seed=40 + L)
    ls = F.synth_labels(3000, 20, 1, 3, 1.0, seed=41)
    res = F.filtered_build(x, ls, F.balanced_label_starts(ls), 32, 64, 64, 750, 32)
    rng = np.random.default_rng(L)
    ql = rng.integers(0, 20, q.shape[0]).astype(np.uint32)
    off, pts = ls.postings()
    starts = []
    for r in range(q.shape[0]):
        carriers = pts[off[ql[r]]:off[ql[r] + 1]]
        m = int(rng.integers(0, 151)) if r % 17 else 0
        lst = list(rng.choice(carriers, size=m)) if carriers.size else []
        if r % 5 == 0:
            lst += [3000, INVALID] + lst[:2]
        starts.append(lst)
    lab = (ls.offsets, ls.labels, ql) if filtered else (None, None, None)
    ids, dd = D.search(x, res.graph, res.degree, starts, q, 10, L, *lab)
    oi, od, _ = O.query_search(x, res.graph, res.degree, starts, q, 10, L, *lab)
    assert np.array_equal(ids, oi) and np.array_equal(dd.view(np.uint32), od.view(np.uint32))
    assert D.last_search_stats()["capped_queries"] == 0


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["u8", "f32"])
@pytest.mark.parametrize("L", [10, 100, 1000])
def test_gpu_search_on_duplicate_rows(kind, L):
    """2000 rows drawn from 15 distinct vectors and queries equal to some of
    them: every result list is a run of equal distances (many of them 0)
    ordered by id alone; ids and distances bit-exact with the oracle."""
    base, _ = make(kind, 15, 32, seed=L + 1)
    rng = np.random.default_rng(L)
    x = np.ascontiguousarray(base[rng.integers(0, 15, 2000)])
    q = np.ascontiguousarray(np.concatenate([base[rng.integers(0, 15, 100)], make(kind, 100, 32, seed=L)[1][:100]]))
    g, d, med = O.vnew2_build(x, 16, 32, 24, 16)
    ids, dd = D.search(x, g, d, med, q, 10, L)
    oi, od, _ = O.query_search(x, g, d, med, q, 10, L)
    assert np.array_equal(ids, oi)
    assert np.array_equal(dd.view(np.uint32), od.view(np.uint32))
