"""The bench's label-filtered diagnostics on toy graphs with known answers
(CPU only): reachability inside the label-induced subgraph, the per-label
subgraph statistics and the reference's cardinality buckets
(tools/prepare_multilabel_workload.py:243-253)."""
import numpy as np

import bench
from dance_amd import INVALID
from dance_amd import filtered as F


def toy():
    """8 points; label 0 on 0-4, label 1 on 4-7. Edges: 0->1->2 (label 0
    chain), 3 isolated inside label 0 (its only edge goes to 5, label 1),
    4 -> 0; label 1: 5->6, 6->7, 4 -> 5."""
    rows = [[0], [0], [0], [0], [0, 1], [1], [1], [1]]
    ls = F.canonical_labels(rows, 2)
    g = np.full((8, 3), INVALID, np.uint32)
    deg = np.zeros(8, np.uint32)
    for u, vs in {0: [1], 1: [2], 3: [5], 4: [0, 5], 5: [6], 6: [7]}.items():
        g[u, :len(vs)] = vs
        deg[u] = len(vs)
    return ls, g, deg


def test_label_reachability():
    ls, g, deg = toy()
    gt = np.array([[1, 2, 3, INVALID], [2, 3, INVALID, INVALID], [6, 7, INVALID, INVALID]], np.uint32)
    ql = np.array([0, 0, 1], np.uint32)
    r = bench.label_reachability(g, deg, ls, ql, [[0], [3], [5]], gt)
    # query 0 from 0 reaches 1, 2 (not 3): 2/3; query 1 from 3: nothing of
    # {2, 3} but 3 itself: 1/2; query 2 from 5 reaches 6, 7: 1
    assert r["mean_reachable_fraction"] == round((2 / 3 + 1 / 2 + 1) / 3, 4)
    assert r["queries_fully_reachable"] == round(1 / 3, 4)
    r2 = bench.label_reachability(g, deg, ls, ql[:1], [[0, 3]], gt[:1])  # a second start covers 3
    assert r2["mean_reachable_fraction"] == 1.0


def test_label_subgraph_stats():
    ls, g, deg = toy()
    s = bench.label_subgraph_stats(g, deg, ls, [0, 1], np.array([0, 5], np.uint32))
    # label 0 carriers 0-4: in-label out-degrees 1, 1, 0, 0, 1 (4 -> 0; 4 -> 5
    # leaves the label); label 1 carriers 4-7: 1 (4 -> 5), 1, 1, 0
    assert s["in_label_out_degree"] == round((3 / 5 + 3 / 4) / 2, 4)
    assert s["carriers_without_in_label_edge"] == round((2 / 5 + 1 / 4) / 2, 4)
    assert s["start_in_label_out_degree"] == 1.0
    # from 0: {0, 1, 2} of 5; from 5: {5, 6, 7} of 4
    assert s["carriers_reachable_from_start"] == round((3 / 5 + 3 / 4) / 2, 4)


def test_cardinality_buckets():
    rows = [[l] for l, k in enumerate([1, 2, 3, 4, 5, 6, 7, 8, 9, 10]) for _ in range(k)]
    ls = F.canonical_labels(rows, 10)
    b = bench.cardinality_buckets(ls, (("P50", 50.0), ("P1", 1.0)), per_bucket=3)
    assert b["P50"]["target_cardinality"] == 5.5
    assert b["P50"]["labels"] == [4, 5, 3]  # |5 - 5.5| = |6 - 5.5|, ties to the smaller label
    assert b["P1"]["labels"] == [0, 1, 2] and b["P1"]["cardinalities"] == [1, 2, 3]
