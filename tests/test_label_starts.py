"""Label starts of the filtered build (CPU only).

build_memory_index picks each label's entry point by Filtered-DiskANN's
load-balanced FindMedoid, the rule upstream DiskANN's
Index::build_filtered_index applies just before the reference's GPU branch
(integrations/dance-diskann-78256bba.patch:20239, consumed at :20288-20296):
25 carriers drawn per label, the least-loaded wins. Upstream DiskANN is not
available offline and draws with rand(); here the draws come from splitmix64
(pinned by its published outputs). dance_amd.filtered.balanced_label_starts
is checked against an independent statement of the rule and against
invariants; the app's output is compared with it in the GPU test of
build_memory_index.
"""
import collections

import numpy as np
import pytest

from dance_amd import INVALID
from dance_amd import filtered as F

MASK = (1 << 64) - 1


def test_splitmix64_known_answers():
    # Vigna's splitmix64 from state 0: the first three outputs
    s, a = F._splitmix64(0)
    s, b = F._splitmix64(s)
    s, c = F._splitmix64(s)
    assert (a, b, c) == (0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F)


def draws(seed):
    """splitmix64 as a generator: state advances by the golden gamma, output
    is the mixed state (written separately from dance_amd.filtered)."""
    state = seed
    while True:
        state = (state + 0x9E3779B97F4A7C15) & MASK
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
        yield z ^ (z >> 31)


def restated_starts(rows, num_labels, universal=None, seed=1, cands=25):
    """Per label in id order: carriers = rows holding the label or the
    universal label (ascending, unique); 25 draws; the first drawn of minimum
    load wins and its load rises."""
    g = draws(seed)
    load = collections.Counter()
    out = []
    for lab in range(num_labels):
        carriers = sorted({i for i, r in enumerate(rows) if lab in r or (universal is not None and universal in r)})
        if not carriers:
            out.append(INVALID)
            continue
        picked = [carriers[next(g) % len(carriers)] for _ in range(cands)]
        low = min(load[p] for p in picked)
        win = next(p for p in picked if load[p] == low)
        load[win] += 1
        out.append(win)
    return out


def random_rows(rng, n, vocab, max_per, universal_every=0):
    rows = []
    for i in range(n):
        lo = 1 if universal_every else 0
        r = sorted(set(int(t) for t in rng.integers(lo, vocab, int(rng.integers(1, max_per + 1)))))
        if universal_every and i % universal_every == 0:
            r = sorted(set(r) | {0})
        rows.append(r)
    return rows


@pytest.mark.parametrize("seed,n,vocab,max_per,universal_every", [(0, 300, 20, 3, 0), (1, 50, 40, 2, 0),
                                                                  (2, 400, 12, 4, 7), (3, 30, 100, 1, 0),
                                                                  (4, 1000, 8, 8, 3)])
def test_balanced_starts_match_restatement(seed, n, vocab, max_per, universal_every):
    rng = np.random.default_rng(seed)
    rows = random_rows(rng, n, vocab, max_per, universal_every)
    ls = F.canonical_labels(rows, vocab)
    uni = 0 if universal_every else INVALID
    for s in (1, 7, 12345):
        got = F.balanced_label_starts(ls, uni, seed=s).tolist()
        assert got == restated_starts(rows, vocab, 0 if universal_every else None, seed=s), s


def test_balanced_starts_invariants():
    rng = np.random.default_rng(5)
    rows = random_rows(rng, 500, 30, 3, 9)
    ls = F.canonical_labels(rows, 31)  # label 30 has no carrier of its own
    st = F.balanced_label_starts(ls, 0, seed=3)
    for lab in range(31):
        assert st[lab] != INVALID  # universal carriers carry every label
        assert lab in rows[st[lab]] or 0 in rows[st[lab]]
    st2 = F.balanced_label_starts(ls, INVALID, seed=3)
    assert st2[30] == INVALID
    for lab in range(30):
        if st2[lab] != INVALID:
            assert lab in rows[st2[lab]]


def test_balanced_starts_spread_the_load():
    """40 labels all carried by the same 8 points: every label's 25 draws
    hold each of the 8 (seed chosen so), so the least-loaded point always
    wins and the loads end at exactly 5 each; the centroid rule would put all
    40 on one point."""
    rows = [list(range(40)) for _ in range(8)] + [[] for _ in range(4)]
    ls = F.canonical_labels(rows, 40)
    st = F.balanced_label_starts(ls, INVALID, seed=1)
    assert set(st.tolist()) <= set(range(8))
    assert sorted(collections.Counter(st.tolist()).values()) == [5] * 8
    x = np.random.default_rng(0).standard_normal((12, 4)).astype(np.float32)
    assert len(set(F.label_starts(x, ls).tolist())) == 1


def py_start_hash(point, label):
    x = ((point << 32) ^ label ^ 0x9E3779B97F4A7C15) & MASK
    x ^= x >> 30
    x = (x * 0xBF58476D1CE4E5B9) & MASK
    x ^= x >> 27
    x = (x * 0x94D049BB133111EB) & MASK
    x ^= x >> 31
    return x & 0xFFFFFFFF


def streamed_extra_starts(rows, num_labels, starts, k):
    """The reference's sampler (patch:19845-19873) restated: points in
    ascending order, each label of the point other than its start's own
    point; keep k (hash, point) samples, a new one replacing the largest when
    its hash is smaller; finally sort the samples."""
    samples = {}
    for loc, r in enumerate(rows):
        for lab in r:
            if lab >= num_labels or starts[lab] == INVALID or starts[lab] == loc:
                continue
            s = samples.setdefault(lab, [])
            h = py_start_hash(loc, lab)
            if len(s) < k:
                s.append((h, loc))
            else:
                worst = max(s)
                if h < worst[0]:
                    s[s.index(worst)] = (h, loc)
    return [[p for _, p in sorted(samples.get(l, []))] for l in range(num_labels)]


@pytest.mark.parametrize("seed,k", [(0, 1), (1, 4), (2, 16), (3, 40)])
def test_extra_starts_match_streamed_sampler(seed, k):
    rng = np.random.default_rng(60 + seed)
    rows = random_rows(rng, 400, 15, 4)
    ls = F.canonical_labels(rows, 16)  # label 15 without carriers
    st = F.balanced_label_starts(ls, INVALID, seed=2)
    got = [e.tolist() for e in F.extra_label_starts(ls, st, k)]
    assert got == streamed_extra_starts(rows, 16, st, min(k, 16))
    pts = np.arange(50, dtype=np.uint64)
    assert F.start_hash(pts, 7).tolist() == [py_start_hash(int(p), 7) for p in pts]


def test_query_starts_select_nearest_extras():
    rng = np.random.default_rng(70)
    rows = random_rows(rng, 300, 6, 2)
    ls = F.canonical_labels(rows, 6)
    x = rng.integers(0, 256, (300, 8)).astype(np.uint8)
    q = rng.integers(0, 256, (20, 8)).astype(np.uint8)
    ql = rng.integers(0, 6, 20).astype(np.uint32)
    st = F.balanced_label_starts(ls, INVALID, seed=1)
    ex = F.extra_label_starts(ls, st, 8)
    every = F.query_starts(x, q, ql, st, ex)
    near = F.query_starts(x, q, ql, st, ex, select=3)
    for r in range(20):
        l = int(ql[r])
        assert every[r] == sorted({int(st[l])} | set(ex[l].tolist()))
        d = {int(p): int(((x[p].astype(int) - q[r].astype(int)) ** 2).sum()) for p in ex[l]}
        want = sorted(d, key=lambda p: (d[p], p))[:3]
        assert near[r] == sorted({int(st[l])} | set(want))
