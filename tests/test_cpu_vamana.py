"""Pins the CPU Vamana baseline (oracle/cpu_baselines.cpp), the comparator of
the recall gate and the timed CPU baseline (CPU only; no GPU).

Upstream DiskANN (the reference's build dependency, commit 78256bba) is not
available offline, so the baseline restates the published algorithm
(Subramanya et al., NeurIPS 2019, Alg. 1-3) with DiskANN's occlude alpha
ladder and graph slack. Each part is checked here against an independent
Python statement of the same rules, written with other data structures
(sets, re-sorted lists, per-candidate maxima recomputed from scratch), on
small integer rows whose distances are exact and full of ties, so that a
wrong boundary (> against >=), an inverted occlusion ratio, a missing ladder
step or a wrong slack changes the result.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

F32 = np.float32


def _dist(x, a, b):
    d = x[a].astype(np.int64) - x[b].astype(np.int64)
    return float(int((d * d).sum()))


def py_robust_prune(x, p, cands, R, alpha, maxc):
    """RobustPrune(p, V) of the paper's Alg. 2 with DiskANN's alpha ladder:
    the candidates sorted by (distance, id), cut to maxc; at levels 1, 1.2,
    1.44, ... (float32 products, up to alpha) a candidate j is kept when no
    candidate kept before it *in sorted order* has d(p, j) / d(i, j) above the
    level (a zero d(i, j) always blocks); at most R kept, in selection order."""
    pool = sorted({(F32(_dist(x, p, c)), int(c)) for c in cands if c != p})[:maxc]
    kept_pos = []
    kept = []
    level = F32(1.0)
    while level <= F32(alpha) and len(kept) < R:
        for j, (dj, idj) in enumerate(pool):
            if len(kept) >= R:
                break
            if j in kept_pos:
                continue
            worst = F32(0.0)
            for i in kept_pos:
                if i >= j:
                    continue
                dij = F32(_dist(x, pool[i][1], idj))
                r = F32(np.finfo(F32).max) if dij == 0 else F32(dj / dij)
                worst = max(worst, r)
            if worst <= level:
                kept_pos.append(j)
                kept.append(idj)
        level = F32(level * F32(1.2))
    return kept


def py_greedy(x, q, neighbours, start, L):
    """Best-first search (paper Alg. 1): the beam is the L nearest of every
    point seen so far by (distance, id); repeatedly expand its nearest
    unexpanded member. Returns (expanded ids in order, final beam ids)."""
    def d(n):
        t = x[n].astype(np.int64) - q.astype(np.int64)
        return F32(float(int((t * t).sum())))
    seen = {start}
    beam = [(d(start), start)]
    done = set()
    order = []
    while True:
        todo = [c for c in beam if c[1] not in done]
        if not todo:
            break
        _, u = todo[0]
        done.add(u)
        order.append(u)
        for n in neighbours(u):
            if n in seen:
                continue
            seen.add(n)
            beam = sorted(beam + [(d(n), n)])[:L]
    return order, [b[1] for b in beam]


def py_vamana(x, R, L, alpha, maxc, keep_own=False):
    """The paper's Alg. 3 as one pass in id order with DiskANN's graph slack:
    search from the start, prune V (DiskANN's code) or V u N_out(p) (the
    paper's Alg. 2, keep_own), then for each new neighbour n append p while n
    holds fewer than ceil(1.3 R) ids, else prune N_out(n) u {p}; rows above R
    are pruned at the end. The start is the point nearest to the centroid
    (fp64, first on ties)."""
    n, dim = x.shape
    cent = [0.0] * dim
    for i in range(n):
        for e in range(dim):
            cent[e] += float(x[i, e])
    cent = [c / n for c in cent]
    start, best = 0, math.inf
    for i in range(n):
        s = 0.0
        for e in range(dim):
            t = float(x[i, e]) - cent[e]
            s += t * t
        if s < best:
            best, start = s, i
    slack = math.ceil(1.3 * R)
    G = [[] for _ in range(n)]
    for p in range(n):
        order, _ = py_greedy(x, x[p], lambda u: list(G[u]), start, L)
        G[p] = py_robust_prune(x, p, order + (G[p] if keep_own else []), R, alpha, maxc)
        for m in G[p]:
            if p in G[m]:
                continue
            if len(G[m]) < slack:
                G[m].append(p)
            else:
                G[m] = py_robust_prune(x, m, G[m] + [p], R, alpha, maxc)
    for m in range(n):
        if len(G[m]) > R:
            G[m] = py_robust_prune(x, m, G[m], R, alpha, maxc)
    return G, start


def tie_rows(rng, n, dim, levels):
    return rng.integers(0, levels, (n, dim)).astype(np.uint8)


@pytest.mark.parametrize("seed,levels,R,alpha,maxc", [(0, 3, 6, 1.2, 750), (1, 2, 4, 1.2, 750),
                                                      (2, 4, 8, 1.5, 750), (3, 3, 5, 1.0, 750),
                                                      (4, 5, 6, 1.2, 9), (5, 3, 12, 2.0, 30)])
def test_occlude_matches_alpha_ladder(seed, levels, R, alpha, maxc):
    rng = np.random.default_rng(seed)
    x = tie_rows(rng, 60, 6, levels)
    for p in range(0, 60, 7):
        cands = rng.choice(60, size=40, replace=False)
        cands = cands[cands != p]
        d = np.array([_dist(x, p, c) for c in cands], np.float32)
        got = O.cpu_occlude(x, cands, d, R, alpha, maxc)
        assert got == py_robust_prune(x, p, cands, R, alpha, maxc), (seed, p)


def test_occlude_ladder_worked_cases():
    """Worked by hand. 1-D rows p=0, a=2, b=4, c=10: d(p, .) = 4, 16, 100;
    b's ratio d(p,b)/d(a,b) = 16/4 = 4, c's 100/64 = 1.5625 (c comes after b,
    so c's selection never counts against b). Levels are 1, 1.2, 1.44, 1.728,
    2.07, 2.49, 2.99, 3.58, 4.30 (float32 powers of 1.2)."""
    x = np.array([[0], [2], [4], [10]], np.uint8)
    d = np.array([4, 16, 100], np.float32)
    assert O.cpu_occlude(x, [1, 2, 3], d, 3, 1.2) == [1]
    assert O.cpu_occlude(x, [1, 2, 3], d, 3, 1.6) == [1]         # c needs level 1.728
    assert O.cpu_occlude(x, [1, 2, 3], d, 3, 1.75) == [1, 3]
    assert O.cpu_occlude(x, [1, 2, 3], d, 3, 4.0) == [1, 3]      # b needs level 4.30
    assert O.cpu_occlude(x, [1, 2, 3], d, 3, 4.3) == [1, 3, 2]
    assert O.cpu_occlude(x, [1, 2, 3], d, 1, 4.3) == [1]         # R caps the list
    # a ratio of exactly the level keeps the candidate: p=(0,0), a=(2,0),
    # b=(1,2): d(p,a) = 4, d(p,b) = 5 = d(a,b)
    y = np.array([[0, 0], [2, 0], [1, 2]], np.uint8)
    assert O.cpu_occlude(y, [1, 2], np.array([4, 5], np.float32), 2, 1.0) == [1, 2]
    # equal rows: d(a,b) = 0 always blocks
    w = np.array([[0], [1], [1]], np.uint8)
    assert O.cpu_occlude(w, [1, 2], np.array([1, 1], np.float32), 2, 10.0) == [1]
    # maxc cuts the sorted list before the ladder
    assert O.cpu_occlude(x, [3, 2, 1], np.array([100, 16, 4], np.float32), 3, 4.3, maxc=2) == [1, 2]
    for alpha in (1.2, 1.6, 1.75, 4.0, 4.3):
        assert O.cpu_occlude(x, [1, 2, 3], d, 3, alpha) == py_robust_prune(x, 0, [1, 2, 3], 3, alpha, 750)


@pytest.mark.parametrize("seed,L", [(0, 500), (1, 500), (2, 12), (3, 5), (4, 30)])
def test_greedy_matches_best_first(seed, L):
    rng = np.random.default_rng(20 + seed)
    n, R = 120, 6
    x = tie_rows(rng, n, 5, 4)
    g = np.full((n, R), 0xFFFFFFFF, np.uint32)
    deg = rng.integers(1, R + 1, n).astype(np.uint32)
    for v in range(n):
        g[v, :deg[v]] = rng.choice(n, size=deg[v], replace=False)
    for qi in range(5):
        q = rng.integers(0, 4, 5).astype(np.uint8)
        start = int(rng.integers(0, n))
        exp, beam = O.cpu_greedy(x, g, deg, start, q, L)
        want_exp, want_beam = py_greedy(x, q, lambda u: [int(t) for t in g[u, :deg[u]]], start, L)
        assert exp == want_exp and beam == want_beam


def test_greedy_with_full_beam_is_exact_on_reachable_points():
    """With L >= N the search expands every point reachable from the start,
    so its beam starts with the exact nearest neighbours (brute force)."""
    rng = np.random.default_rng(7)
    n = 200
    x = rng.integers(0, 255, (n, 8)).astype(np.uint8)
    g = np.stack([np.roll(np.arange(n), -k - 1) for k in range(3)], 1).astype(np.uint32)  # a ring: connected
    deg = np.full(n, 3, np.uint32)
    q = rng.integers(0, 255, 8).astype(np.uint8)
    exp, beam = O.cpu_greedy(x, g, deg, 0, q, n)
    assert sorted(exp) == list(range(n))
    d = ((x.astype(np.int64) - q.astype(np.int64)) ** 2).sum(1)
    assert beam[:10] == [int(i) for i in np.lexsort((np.arange(n), d))[:10]]


@pytest.mark.parametrize("seed,n,dim,levels,R,L,alpha,maxc", [
    (0, 150, 6, 4, 8, 16, 1.2, 750), (1, 120, 4, 3, 6, 10, 1.2, 750),
    (2, 160, 8, 6, 10, 20, 1.5, 40), (3, 100, 5, 2, 5, 8, 1.0, 750), (5, 1000, 8, 6, 8, 8, 1.2, 750)])
@pytest.mark.parametrize("pool", ["diskann", "paper"])
def test_single_thread_build_matches_restatement(seed, n, dim, levels, R, L, alpha, maxc, pool):
    rng = np.random.default_rng(40 + seed)
    x = tie_rows(rng, n, dim, levels)
    g, deg, start = O.cpu_vamana_build(x, R, L, alpha, maxc, threads=1, pool=pool)
    G, s2 = py_vamana(x, R, L, alpha, maxc, keep_own=pool == "paper")
    assert start == s2
    for v in range(n):
        assert g[v, :deg[v]].tolist() == G[v], v
        assert np.all(g[v, deg[v]:] == 0xFFFFFFFF)



def test_parallel_build_is_a_valid_graph():
    """Many threads: the graph depends on thread timing, but every row holds
    distinct valid non-self ids, at most R of them, and search reaches high
    recall."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3000, 16)).astype(np.float32)
    g, deg, start = O.cpu_vamana_build(x, 16, 32, 1.2, 750, threads=4)
    for v in range(3000):
        row = g[v, :deg[v]].tolist()
        assert 1 <= len(row) <= 16 and len(set(row)) == len(row) and v not in row and max(row) < 3000
    q = rng.standard_normal((100, 16)).astype(np.float32)
    gt, _ = O.bruteforce_knn(x, q, 10)
    assert O.recall_at_k(O.beam_search(x, g, deg, start, q, 10, 64), gt) > 0.95


def test_pools_differ():
    """The two candidate pools give different graphs once points receive
    reverse edges before their own turn (a build that ignored the setting
    would pass the restatement test of only one of them)."""
    rng = np.random.default_rng(45)
    x = tie_rows(rng, 1000, 8, 6)  # a beam of 8: searches often miss earlier reverse edges
    g1, d1, _ = O.cpu_vamana_build(x, 8, 8, 1.2, 750, threads=1, pool="diskann")
    g2, d2, _ = O.cpu_vamana_build(x, 8, 8, 1.2, 750, threads=1, pool="paper")
    assert not (np.array_equal(g1, g2) and np.array_equal(d1, d2))
