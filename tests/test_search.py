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


def test_search_parameter_errors():
    x = np.zeros((10, 4), np.float32)
    g = np.zeros((10, 4), np.uint32)
    deg = np.zeros(10, np.uint32)
    for k, L in [(0, 10), (65, 100), (10, 5), (10, 257)]:
        with pytest.raises(D.BuildError):
            D.search(x, g, deg, 0, x[:2], k, L)
    with pytest.raises(D.BuildError):  # partial label filter
        D.search(x, g, deg, 0, x[:2], 4, 8, label_offsets=np.zeros(11, np.uint32))


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
@pytest.mark.parametrize("L", [10, 64, 100, 200])
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
