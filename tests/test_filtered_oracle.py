"""Pins the CPU oracle of the filtered build (oracle/filtered_oracle.cpp) with
checks that do not restate its code: closed forms, an independent greedy
formulation of FilteredRobustPrune, dictionary-based merges, special cases
that reduce to textbook RobustPrune, and build invariants. CPU only."""
import numpy as np
import pytest

from dance_amd import INVALID
from dance_amd import filtered as F
from oracle import oracle as O

FMAX = np.float32(np.finfo(np.float32).max)


def sqdist(x, a, b):
    d = x[a].astype(np.float64) - x[b].astype(np.float64)
    return float((d * d).sum())


def test_random_backbone_closed_form():
    for N, R in [(1, 8), (2, 8), (17, 32), (500, 32), (3000, 8)]:
        g, d = O.filtered_random_graph(N, R)
        target = min(16, R, N - 1)
        assert (d == target).all()
        for row in range(0, N, max(1, N // 50)):
            nb = g[row, :target]
            assert len(set(nb.tolist())) == target and row not in nb and (nb < N).all()
            assert (g[row, target:] == INVALID).all()
            if target == 0:
                continue
            # first entry: the first hash draw (attempt 0, 1, ...) that is not the row
            a = 0
            while True:
                h = O.hash_u32(((row * 0x9E3779B1) ^ (42 * 0x85EBCA6B) ^ (a * 0xC2B2AE35)) & 0xFFFFFFFF) % N
                if h != row:
                    break
                a += 1
            assert nb[0] == h


def labels_of(ls, i):
    return set(ls.row(i).tolist())


def greedy_prune(x, ls, row, ids, ds, R, alpha):
    """FilteredRobustPrune as a single pass in (distance, id) order: a
    candidate is kept iff no already-kept p occludes it, where p occludes c
    iff (F_row & F_c) <= F_p, d(p,c) > 0 and alpha * d(p,c) <= d(row,c)."""
    order = sorted(range(len(ids)), key=lambda i: (ds[i], ids[i], i))
    kept = []
    fr = labels_of(ls, row)
    for i in order:
        if len(kept) == R:
            break
        c = int(ids[i])
        occluded = False
        for p in kept:
            if (fr & labels_of(ls, c)) <= labels_of(ls, p):
                pd = np.float32(O.distance(x, p, c))
                if pd > 0 and np.float32(alpha) * pd <= ds[i]:
                    occluded = True
                    break
        if not occluded:
            kept.append(c)
    return kept


@pytest.mark.parametrize("seed", [1, 2, 3])
@pytest.mark.parametrize("vocab", [1, 4, 12])
def test_filtered_prune_matches_greedy(seed, vocab):
    rng = np.random.default_rng(seed)
    n = 400
    x = rng.integers(0, 256, (n, 16), dtype=np.uint8)
    x[7] = x[3]  # a zero-distance pair (pd > 0 rule)
    ls = F.synth_labels(n, vocab, 1, min(3, vocab), 1.0, seed=seed)
    for row in (0, 3, 11, 250):
        ids = rng.choice(np.setdiff1d(np.arange(n), [row]), 120, replace=False).astype(np.uint32)
        if row == 3:
            ids[0] = 7
        ds = np.array([O.distance(x, row, int(c)) for c in ids], np.float32)
        for R, alpha in [(32, 1.2), (16, 1.0), (120, 1.2)]:
            got = O.filtered_prune(x, ls.offsets, ls.labels, row, ids, ds, R, alpha).tolist()
            assert got == greedy_prune(x, ls, row, ids, ds, R, alpha)


def test_single_label_prune_is_textbook_robust_prune():
    """With one label everywhere the coverage test always passes: the result is
    DiskANN's RobustPrune (Alg. 2) without the degree fill, computed on exact
    fp64 distances of integer vectors (exact in fp32 at this size)."""
    rng = np.random.default_rng(4)
    x = rng.integers(0, 256, (300, 12), dtype=np.uint8)
    ls = F.canonical_labels([[5]] * 300, 8)
    ids = np.arange(1, 300, dtype=np.uint32)
    ds = np.array([sqdist(x, 0, int(c)) for c in ids], np.float32)
    cand = {int(c): float(d) for c, d in zip(ids, ds)}
    out = []
    while cand and len(out) < 24:
        p = min(cand, key=lambda c: (cand[c], c))
        out.append(p)
        del cand[p]
        for c in list(cand):
            pd = sqdist(x, p, c)
            if pd > 0 and np.float32(1.2) * np.float32(pd) <= np.float32(cand[c]):
                del cand[c]
    got = O.filtered_prune(x, ls.offsets, ls.labels, 0, ids, ds, 24, 1.2).tolist()
    assert got == out


def dict_merge(row, N, C_, streams):
    """Insertion-ordered dict: a repeat keeps the smaller distance; once C_
    entries are held every further candidate is ignored, repeats included
    (reference canonical_merge_one_warp, gpu_vamana_filtered.cu:4677-4678)."""
    out = {}
    for c, d in streams:
        if c >= N or c == row or len(out) >= C_:
            continue
        out[c] = min(out.get(c, d), d)
    return list(out.keys()), list(out.values())


def merge_inputs(rng, N, R, ls, row, keep, nord):
    T = ls.labels.shape[0]
    tids = rng.integers(0, N + 3, (T, keep)).astype(np.uint32)  # includes invalid ids
    tids[rng.random((T, keep)) < 0.2] = INVALID
    td = rng.random((T, keep)).astype(np.float32)
    graph = rng.integers(0, N, (N, R)).astype(np.uint32)
    deg = rng.integers(0, R + 1, N).astype(np.uint32)
    oid = rng.integers(0, N, nord).astype(np.uint32)
    od = rng.random(nord).astype(np.float32)
    return tids, td, graph, deg, oid, od


def test_merge_without_quota_is_ordered_min_dedupe():
    """Rows with 0 or more than 16 labels: tasks, label-sharing old neighbours
    (distance FLT_MAX), union results; first position kept, minimum distance."""
    rng = np.random.default_rng(7)
    N, R, keep = 60, 8, 4
    rows = [list(rng.choice(20, rng.integers(1, 4), replace=False)) for _ in range(N)]
    rows[5] = []
    rows[9] = list(range(18))
    ls = F.canonical_labels(rows, 20)
    for row, C_ in [(5, 128), (9, 128), (9, 10)]:
        tids, td, graph, deg, oid, od = merge_inputs(rng, N, R, ls, row, keep, 8)
        got_i, got_d = O.filtered_merge(N, R, C_, keep, ls.offsets, ls.labels, 20, graph, deg, row, tids, td, oid, od)
        streams = []
        for p in range(ls.offsets[row], ls.offsets[row + 1]):
            streams += [(int(tids[p, i]), float(td[p, i])) for i in range(keep)]
        fr = labels_of(ls, row)
        for i in range(min(int(deg[row]), R)):
            c = int(graph[row, i])
            if c < N and c != row and fr & labels_of(ls, c):
                streams.append((c, float(FMAX)))
        streams += [(int(c), float(d)) for c, d in zip(oid, od)]
        want_i, want_d = dict_merge(row, N, C_, streams)
        assert got_i.tolist() == want_i
        assert np.array_equal(got_d, np.array(want_d, np.float32))


def test_merge_single_label_quota():
    """One row label: quota = max(R, keep); the kept list is the first quota
    merged candidates that carry the row's label, in merged order."""
    rng = np.random.default_rng(8)
    N, R, keep = 300, 16, 8
    rows = [[int(rng.integers(0, 3))] for _ in range(N)]
    rows[1] = [2]
    ls = F.canonical_labels(rows, 3)
    tids, td, graph, deg, oid, od = merge_inputs(rng, N, R, ls, 1, keep, 64)
    got_i, _ = O.filtered_merge(N, R, 128, keep, ls.offsets, ls.labels, 3, graph, deg, 1, tids, td, oid, od)
    streams = [(int(tids[0 + ls.offsets[1], i]), 0.0) for i in range(keep)]
    for i in range(min(int(deg[1]), R)):
        c = int(graph[1, i])
        if c < N and c != 1 and rows[c][0] == 2:
            streams.append((c, 0.0))
    streams += [(int(c), 0.0) for c in oid]
    merged, _ = dict_merge(1, N, 128, streams)
    want = [c for c in merged if rows[c][0] == 2][:max(R, keep)]
    assert got_i.tolist() == want


def test_build_invariants_and_determinism():
    rng = np.random.default_rng(3)
    N = 2000
    x = rng.integers(0, 256, (N, 32), dtype=np.uint8)
    ls = F.synth_labels(N, 30, 1, 4, 1.0, seed=4)
    st, gs = F.label_starts(x, ls), F.global_start(x)
    rc, g, d, diag = O.filtered_build(x, ls.offsets, ls.labels, st, 30, 32, 64, 64, 750, 32, 1.2, INVALID, gs)
    assert rc == 0
    assert diag[0] == 0 and diag[1] == 0            # invalid, self
    assert diag[10] == 0                              # every edge shares a label with its row
    assert diag[7] == d.sum() and d.max() <= 32
    for row in range(N):
        nb = g[row, :d[row]]
        assert len(set(nb.tolist())) == d[row]
        assert (g[row, d[row]:] == INVALID).all()
    rc2, g2, d2, _ = O.filtered_build(x, ls.offsets, ls.labels, st, 30, 32, 64, 64, 750, 32, 1.2, INVALID, gs)
    assert np.array_equal(g, g2) and np.array_equal(d, d2)


def test_round_log_changed_rows():
    """The per-round changed count equals the number of rows whose neighbour
    set differs between the graphs after r and r + 1 rounds (builds of 0..3
    rounds are prefixes of one another); touched rows are at most the reverse
    proposals, which are at most the edges of a forward graph."""
    rng = np.random.default_rng(8)
    N, R = 1200, 24
    x = rng.integers(0, 256, (N, 32), dtype=np.uint8)
    ls = F.synth_labels(N, 20, 1, 3, 1.0, seed=9)
    st, gs = F.label_starts(x, ls), F.global_start(x)
    graphs = []
    for rounds in range(4):
        rc, g, d, _ = O.filtered_build(x, ls.offsets, ls.labels, st, 20, R, 48, 48, 750, 24, 1.2, INVALID, gs,
                                       rounds=rounds)
        assert rc == 0
        graphs.append([set(g[r, :d[r]].tolist()) for r in range(N)])
    log = O.filtered_round_log()
    for r in range(3):
        changed = sum(1 for v in range(N) if graphs[r][v] != graphs[r + 1][v])
        assert log[r, 0] == changed
        assert 0 < log[r, 1] <= log[r, 2] <= N * R
    O.filtered_build(x, ls.offsets, ls.labels, st, 20, R, 48, 48, 750, 24, 1.2, INVALID, gs, rounds=1)
    log1 = O.filtered_round_log()
    assert np.array_equal(log1[0], log[0]) and not log1[1:].any()


def test_build_parameter_errors():
    x = np.zeros((10, 4), np.uint8)
    ls = F.canonical_labels([[0]] * 10, 1)
    st = np.zeros(1, np.uint32)
    assert O.filtered_build(x, ls.offsets, ls.labels, st, 1, R=8, C_=4)[0] == -1
    assert O.filtered_build(x, ls.offsets, ls.labels, st, 1, R=70, C_=750)[0] == 1
    assert O.filtered_build(x, ls.offsets, ls.labels, st, 1, R=8, C_=64, rounds=4)[0] == -1


def shortlist_by_sorting(row_labels, labels_of, label_size, universal, num_labels, R, ids, ds):
    """The rare-label shortlist restated with sorted lists: per eligible row
    label, its quota smallest (distance, id, position) carriers in order, each
    output once; then the smallest remaining fill up to R."""
    cand = [(float(d), int(i), p) for p, (i, d) in enumerate(zip(ids, ds)) if i != INVALID and d <= FMAX]
    out, taken = [], set()
    quota = max(1, R // len(row_labels)) if row_labels else 0
    for label in row_labels:
        if label == universal or label >= num_labels or label_size[label] > R * R:
            continue
        for d, i, p in sorted(x for x in cand if label in labels_of(x[1]))[:quota]:
            if len(out) >= R:
                break
            if p not in taken:
                taken.add(p)
                out.append((i, d))
    for d, i, p in sorted(cand):
        if len(out) >= R:
            break
        if p not in taken:
            taken.add(p)
            out.append((i, d))
    return out


@pytest.mark.parametrize("seed", range(12))
def test_rare_shortlist_matches_sorted_restatement(seed):
    rng = np.random.default_rng(seed)
    N, vocab = 60, 10
    rows = [sorted(set(int(v) for v in rng.choice(vocab + 2, int(rng.integers(0, 5)), replace=False)))
            for _ in range(N)]
    offs = np.zeros(N + 1, np.uint32)
    offs[1:] = np.cumsum([len(r) for r in rows])
    labs = np.array([v for r in rows for v in r], np.uint32)
    universal = int(rng.integers(0, vocab)) if seed % 3 == 0 else INVALID
    size = {l: sum(l in r for r in rows) for l in range(vocab + 2)}
    R = int(rng.integers(2, 12))
    row = int(rng.integers(0, N))
    n = int(rng.integers(0, 40))
    ids = rng.integers(0, N, n).astype(np.uint32)
    ids[rng.random(n) < 0.1] = INVALID
    for k in range(1, n):  # repeated ids: each position is taken at most once
        if rng.random() < 0.1:
            ids[k] = ids[k - 1]
    ds = rng.integers(0, 6, n).astype(np.float32)  # many ties
    ds[rng.random(n) < 0.05] = FMAX
    got_i, got_d = O.filtered_shortlist(offs, labs, vocab, universal, R, row, ids, ds)
    want = shortlist_by_sorting(rows[row], lambda i: rows[i], size, universal, vocab, R, ids, ds)
    assert list(zip(got_i.tolist(), got_d.tolist())) == [(i, d) for i, d in want]


def publish_by_composition(x, ls, universal, g, d, R, PR, alpha):
    """The publish step restated from its two pinned parts (the shortlist and
    FilteredRobustPrune): every row's R-row distanced, shortlisted and pruned
    to PR; then rows with reverse edges in that graph rebuilt from their row
    plus the new sources (not the row itself), distanced again, shortlisted
    and pruned to PR."""
    N = x.shape[0]

    def one(row, ids):
        ids = np.asarray(ids, np.uint32)
        ds = np.array([O.distance(x, row, int(c)) for c in ids], np.float32)
        si, sd = O.filtered_shortlist(ls.offsets, ls.labels, ls.num_labels, universal, PR, row, ids, ds)
        return O.filtered_prune(x, ls.offsets, ls.labels, row, si, sd, PR, alpha).tolist()

    fwd = [one(row, g[row, :min(int(d[row]), R)]) for row in range(N)]
    rev = [[] for _ in range(N)]
    for row in range(N):
        for c in fwd[row]:
            if c < N and c != row:
                rev[c].append(row)
    out = [one(row, fwd[row] + [s for s in rev[row] if s not in fwd[row] and s != row]) if rev[row] else fwd[row]
           for row in range(N)]
    pg = np.full((N, PR), INVALID, np.uint32)
    for row, r in enumerate(out):
        pg[row, :len(r)] = r
    return pg, np.array([len(r) for r in out], np.uint32)


@pytest.mark.parametrize("PR,universal", [(6, INVALID), (20, 0), (31, INVALID)])
def test_publish_matches_composition(PR, universal):
    rng = np.random.default_rng(PR)
    N, R = 400, 32
    x = rng.integers(0, 256, (N, 16), dtype=np.uint8)
    ls = F.synth_labels(N, 12, 1, 4, 1.0, seed=PR + 1)
    st, gs = F.label_starts(x, ls), F.global_start(x)
    args = (x, ls.offsets, ls.labels, st, 12, R, 48, 48, 750, 32, 1.2, universal, gs)
    rc, g, d, _ = O.filtered_build(*args)
    assert rc == 0
    rc, pg, pd, diag = O.filtered_build(*args, publish_R=PR)
    assert rc == 0 and pg.shape == (N, PR)
    want_g, want_d = publish_by_composition(x, ls, universal, g, d, R, PR, 1.2)
    assert np.array_equal(pd, want_d)
    assert np.array_equal(pg, want_g)
    assert diag[7] == pd.sum() and pd.max() <= PR
    # at or above R the publish step does nothing
    rc, g2, d2, _ = O.filtered_build(*args, publish_R=R)
    assert rc == 0 and np.array_equal(g2, g) and np.array_equal(d2, d)


# ------------------------------------------------- task and union searches

def search_case(seed, N=160, dim=4, vocab=6, R=6):
    """Small-integer rows (exact, frequently tied distances), 1-3 labels per
    point, a random graph with invalid and self entries, label starts."""
    rng = np.random.default_rng(seed)
    x = rng.integers(0, 4, (N, dim)).astype(np.uint8)
    rows = [list(rng.choice(vocab, int(rng.integers(1, 4)), replace=False)) for _ in range(N)]
    ls = F.canonical_labels(rows, vocab)
    graph = rng.integers(0, N, (N, R)).astype(np.uint32)
    graph[rng.random((N, R)) < 0.05] = INVALID
    for v in range(0, N, 17):
        graph[v, 0] = v  # self entries are skipped
    deg = rng.integers(0, R + 1, N).astype(np.uint32)
    starts = F.label_starts(x, ls)
    return x, ls, graph, deg, starts


def best_first_slots(x, row, seeds, admissible, graph, deg, cap, steps):
    """The canonical pool of filtered.cu:4156-4263, restated with Python
    lists: slots in insertion order; an id already present keeps its slot
    (its distance can only be the same); a new id is appended while there is
    room, else replaces the slot of the worst (distance, id) if it is better;
    each step expands the unexpanded slot of smallest (distance, id).
    `seeds` are inserted first, in order; expansions insert the admissible
    neighbours. Returns the slots as (id, distance)."""
    N, R = graph.shape
    slots = []  # [id, distance, expanded]

    def offer(v):
        if any(s[0] == v for s in slots):
            return
        d = np.float32(O.distance(x, row, v))
        if len(slots) < cap:
            slots.append([v, d, False])
            return
        w = max(range(len(slots)), key=lambda p: (slots[p][1], slots[p][0]))
        if (d, v) < (slots[w][1], slots[w][0]):
            slots[w] = [v, d, False]

    for v in seeds:
        offer(v)
    for _ in range(steps):
        open_ = [p for p in range(len(slots)) if not slots[p][2]]
        if not open_:
            break
        p = min(open_, key=lambda q: (slots[q][1], slots[q][0]))
        slots[p][2] = True
        e = slots[p][0]
        for j in range(min(int(deg[e]), R)):
            v = int(graph[e, j])
            if v < N and v != row and admissible(v):
                offer(v)
    return [(s[0], s[1]) for s in slots]


def label_seeds(ls, row, label, count):
    """Posting-list seeds h(row + s*7919 + label*17) mod |P(label)|, in s order."""
    off, pts = ls.postings()
    pc = int(off[label + 1] - off[label])
    out = []
    for s in range(min(count, pc)):
        out.append(int(pts[off[label] + O.hash_u32((row + s * 7919 + label * 17) & 0xFFFFFFFF) % pc]))
    return out


@pytest.mark.parametrize("seed", [1, 2])
@pytest.mark.parametrize("cap", [8, 32, 200])
def test_task_search_matches_restated_pool(seed, cap):
    """canonical_filtered_task_search (filtered.cu:4265-4426): start, up to 16
    posting seeds, the row's label-carrying neighbours, then 64 expansions
    over label carriers; the first `keep` slots are emitted. cap 200 holds
    every carrier (no eviction: the emitted ids are the first eight distinct
    ids in insertion order); caps 8 and 32 evict."""
    x, ls, graph, deg, starts = search_case(seed)
    N = x.shape[0]
    keep = 8
    for row in range(0, N, 7):
        for label in ls.row(row).tolist() + [int(ls.num_labels), 0]:
            got_i, got_d = O.filtered_task_search(x, ls.offsets, ls.labels, starts, ls.num_labels, INVALID, graph,
                                                  deg, row, label, cap, keep, 64)
            if label >= ls.num_labels:
                assert (got_i == INVALID).all() and (got_d == FMAX).all()
                continue
            carriers = labels_of

            def admissible(v, label=label):
                return label in carriers(ls, v)
            seeds = []
            st = int(starts[label])
            if st < N and st != row:
                seeds.append(st)
            seeds += [v for v in label_seeds(ls, row, label, 16) if v != row]
            seeds += [int(v) for v in graph[row, :min(int(deg[row]), graph.shape[1])]
                      if v < N and v != row and admissible(int(v))]
            slots = best_first_slots(x, row, seeds, admissible, graph, deg, cap, 64)
            want = slots[:keep] + [(INVALID, FMAX)] * (keep - min(keep, len(slots)))
            assert got_i.tolist() == [w[0] for w in want], (row, label)
            assert np.array_equal(got_d, np.array([w[1] for w in want], np.float32))


def test_task_search_universal_label_emits_nothing():
    x, ls, graph, deg, starts = search_case(3)
    got_i, _ = O.filtered_task_search(x, ls.offsets, ls.labels, starts, ls.num_labels, 2, graph, deg, 5, 2, 32, 8,
                                      64)
    assert (got_i == INVALID).all()


@pytest.mark.parametrize("seed", [4, 5])
@pytest.mark.parametrize("cap", [16, 64, 400])
def test_union_search_matches_restated_pool(seed, cap):
    """canonical_ordinary_search (filtered.cu:4529-4670): per row label its
    start and up to 64 posting seeds, the global start when it shares a row
    label, the row's compatible neighbours, 64 expansions over points sharing
    a row label; the first `keep` slots are emitted (INVALID past the pool)."""
    x, ls, graph, deg, starts = search_case(seed, N=240)
    N = x.shape[0]
    keep = 64
    gstart = F.global_start(x)
    for row in range(0, N, 11):
        fr = labels_of(ls, row)

        def admissible(v, fr=fr):
            return bool(fr & labels_of(ls, v))
        seeds = []
        for label in ls.row(row).tolist():
            st = int(starts[label])
            if st < N and st != row:
                seeds.append(st)
            seeds += [v for v in label_seeds(ls, row, label, 64) if v != row]
        if gstart != row and admissible(gstart):
            seeds.append(gstart)
        seeds += [int(v) for v in graph[row, :min(int(deg[row]), graph.shape[1])]
                  if v < N and v != row and admissible(int(v))]
        slots = best_first_slots(x, row, seeds, admissible, graph, deg, cap, 64)
        got_i, got_d = O.filtered_ordinary_search(x, ls.offsets, ls.labels, starts, ls.num_labels, graph, deg, row,
                                                  cap, keep, 64, gstart)
        want = slots[:keep] + [(INVALID, FMAX)] * (keep - min(keep, len(slots)))
        assert got_i.tolist() == [w[0] for w in want], row
        assert np.array_equal(got_d, np.array([w[1] for w in want], np.float32))


# ------------------------------------------------- label quota, many labels

def brute_force_quota(ls, row, merged, R, keep):
    """Label-quota compaction (filtered.cu:4703-4842) restated with Python
    sets: each merged candidate, in order, takes the row label it carries
    with the fewest points (ties: smaller label id) among labels whose count
    is below quota = max(ceil(R / |F_row|), keep), or is dropped; rows with
    no label or more than 16 keep the merged list as it is."""
    off, _ = ls.postings()
    card = {l: int(off[l + 1] - off[l]) for l in range(ls.num_labels)}
    fr = sorted(ls.row(row).tolist())
    if not (1 <= len(fr) <= 16):
        return merged
    quota = max(-(-R // len(fr)), keep)
    counts = {l: 0 for l in fr}
    kept = []
    for c in merged:
        options = [l for l in fr if l in labels_of(ls, c) and counts[l] < quota]
        if not options:
            continue
        best = min(options, key=lambda l: (card[l], l))
        counts[best] += 1
        kept.append(c)
    assert all(v <= quota for v in counts.values())
    return kept


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_merge_multi_label_quota_with_cardinality_ties(seed):
    """Rows with 2..16 labels, several labels of equal posting size (ties go
    to the smaller label id), small quotas that fill up and drop candidates."""
    rng = np.random.default_rng(40 + seed)
    N, R, keep, vocab = 400, 12, 2, 18
    # labels 0..5 get exactly 40 carriers each (cardinality ties), the rest random
    rows = [[] for _ in range(N)]
    for l in range(6):
        for v in rng.choice(N, 40, replace=False):
            rows[v].append(l)
    for v in range(N):
        rows[v] += list(rng.choice(np.arange(6, vocab), int(rng.integers(0, 4)), replace=False))
        if not rows[v]:
            rows[v] = [6]
    rows[3] = list(range(16))           # 16 labels: quota applies
    rows[4] = list(range(17))           # 17 labels: no quota
    rows[5] = [0, 1, 2]                 # three tied labels
    ls = F.canonical_labels(rows, vocab)
    for row in [3, 4, 5] + list(range(6, 60)):
        tids, td, graph, deg, oid, od = merge_inputs(rng, N, R, ls, row, keep, 96)
        got_i, _ = O.filtered_merge(N, R, 128, keep, ls.offsets, ls.labels, vocab, graph, deg, row, tids, td, oid,
                                    od)
        streams = []
        for p in range(ls.offsets[row], ls.offsets[row + 1]):
            streams += [(int(tids[p, i]), float(td[p, i])) for i in range(keep)]
        fr = labels_of(ls, row)
        for i in range(min(int(deg[row]), R)):
            c = int(graph[row, i])
            if c < N and c != row and fr & labels_of(ls, c):
                streams.append((c, float(FMAX)))
        streams += [(int(c), float(d)) for c, d in zip(oid, od)]
        merged, _ = dict_merge(row, N, 128, streams)
        assert got_i.tolist() == brute_force_quota(ls, row, merged, R, keep), row
