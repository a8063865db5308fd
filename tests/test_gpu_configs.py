"""The BASELINE configurations, built on the GPU through the C ABI.

c1 and c2 at their full 100k and 1M (c1 also with 5 iterations, the setting
that passes c1's recall gate), the c3 and c4 generators at 200k, the c5 filtered build
at 50k and the c5 stitched build at its full 1M: the device graph must equal
the CPU oracle's graph on the same generator output. The oracle graphs are
committed as SHA-256 digests (tests/golden/config_fixtures.json, written by
tests/golden/make_config_fixtures.py), together with a digest of each
input, so that a mismatch tells a changed input from a changed graph.

At full size (c3, c4 at 10M; c5 filtered at 1M) the graphs are checked for
what any correct build guarantees: every listed neighbour is a valid id, not
the row itself and not repeated; rows are INVALID-padded past the degree;
degree <= R; filtered edges share a label with their row; and two builds
are identical (the build is deterministic).
"""
import hashlib
import json
import os

import numpy as np
import pytest

import dance_amd as D
from dance_amd import INVALID
from dance_amd import filtered as F

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(HERE, "golden", "config_fixtures.json")) as _f:
    FIX = json.load(_f)

C5 = dict(dim=192, centers=1024, sigma=0.3, vocab=20_000, R=64, L=100, FL=100, C=750, STEPS=64, alpha=1.2,
          parts=100, Rsmall=32, Lsmall=100, Rstitched=64, Cs=96)


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode() + str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def check_rows(graph, degree, N, R, self_ids=None, min_degree=1):
    """Valid, non-self, unique neighbours before the degree; INVALID after.
    A filtered build may leave a row empty (a point sharing no label with any
    other), so its callers pass min_degree=0."""
    import torch
    dev = torch.device("cuda:0")
    g = torch.from_numpy(graph.view(np.int32)).to(dev).long() & 0xFFFFFFFF
    d = torch.from_numpy(degree.astype(np.int64)).to(dev)
    assert int(d.max()) <= R and int(d.min()) >= min_degree
    col = torch.arange(R, device=dev)[None, :]
    live = col < d[:, None]
    rows = torch.arange(N, device=dev)[:, None] if self_ids is None else torch.from_numpy(self_ids).to(dev)[:, None]
    assert int((live & (g >= N)).sum()) == 0, "invalid neighbour id"
    assert int((~live & (g != INVALID)).sum()) == 0, "row not INVALID-padded past its degree"
    assert int((live & (g == rows)).sum()) == 0, "self loop"
    # padding slots become distinct negative values, so only a repeated
    # neighbour can equal its sorted successor
    s = torch.sort(torch.where(live, g, (-col - 1).expand_as(g)), dim=1).values
    assert int((s[:, 1:] == s[:, :-1]).sum()) == 0, "duplicate neighbour"
    return g, d


# ----------------------------------------------------------------- standard

def standard_input(name, n):
    base, _ = D.make_workload(D.CONFIGS[name], n=n)
    return base


@pytest.mark.parametrize("case", ["c1_100k", "c1_100k_iters5", "c2_1m", "c3_200k", "c4_200k"])
def test_standard_config_equals_oracle(case, monkeypatch):
    fx = FIX[case]
    cfg = D.CONFIGS[fx["config"]]
    base = standard_input(fx["config"], fx["n"])
    assert digest(base) == fx["input"], "generator output changed"
    monkeypatch.setenv("DANCE_VAMANA_ITERS", str(fx.get("iters", 4)))
    res = D.vamana_build(base, cfg["R"], cfg["L"], cfg["C"], cfg["STEPS"])
    print(f"[{case}] medoid {res.medoid} (oracle {fx['medoid']}), degree sum {int(res.degree.sum())} "
          f"(oracle {fx['degree_sum']})", flush=True)
    assert res.medoid == fx["medoid"]
    assert int(res.degree.sum()) == fx["degree_sum"]
    assert digest(res.graph, res.degree, np.array([res.medoid], np.uint32)) == fx["graph"]
    check_rows(res.graph, res.degree, fx["n"], cfg["R"])


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_full_size_graph_invariants_and_determinism(name):
    cfg = D.CONFIGS[name]
    base = standard_input(name, cfg["n"])
    first = D.vamana_build(base, cfg["R"], cfg["L"], cfg["C"], cfg["STEPS"])
    print(f"[{name}] first build {first.stats['gpu_build_seconds']:.2f} s", flush=True)
    assert first.medoid < cfg["n"]
    check_rows(first.graph, first.degree, cfg["n"], cfg["R"])
    h1 = digest(first.graph, first.degree)
    del first
    second = D.vamana_build(base, cfg["R"], cfg["L"], cfg["C"], cfg["STEPS"])
    assert digest(second.graph, second.degree) == h1, "two builds of the same input differ"


# ----------------------------------------------------------------- filtered

def c5_input(n):
    x = D.synth_u8(42, 0, n, C5["dim"], C5["centers"], C5["sigma"])
    ls = F.synth_labels(n, C5["vocab"], 1, 8, 1.0, seed=42)
    return x, ls


def test_c5_filtered_equals_oracle():
    fx = FIX["c5f_50k"]
    x, ls = c5_input(fx["n"])
    starts = F.label_starts(x, ls)
    gs = F.global_start(x)
    assert digest(x, ls.offsets, ls.labels, starts, np.array([gs], np.uint32)) == fx["input"]
    res = F.filtered_build(x, ls, starts, C5["R"], C5["L"], C5["FL"], C5["C"], C5["STEPS"], C5["alpha"],
                           INVALID, gs)
    print(f"[c5f_50k] degree sum {int(res.degree.sum())} (oracle {fx['degree_sum']})", flush=True)
    assert int(res.degree.sum()) == fx["degree_sum"]
    assert digest(res.graph, res.degree) == fx["graph"]
    st = res.stats
    diag = fx["diagnostics"]
    assert (st["invalid_neighbor_count"], st["self_loop_count"]) == (diag[0], diag[1]) == (0, 0)
    assert (st["out_degree_min"], st["out_degree_max"]) == (diag[3], diag[4])


def test_c5_filtered_full_size_label_invariants():
    import torch
    n = 1_000_000
    x, ls = c5_input(n)
    starts = F.label_starts(x, ls)
    gs = F.global_start(x)
    res = F.filtered_build(x, ls, starts, C5["R"], C5["L"], C5["FL"], C5["C"], C5["STEPS"], C5["alpha"],
                           INVALID, gs)
    g, d = check_rows(res.graph, res.degree, n, C5["R"], min_degree=0)
    assert res.stats["invalid_neighbor_count"] == 0 and res.stats["self_loop_count"] == 0
    # every edge (u, v) shares a label: some label of u is a label of v,
    # looked up as the key v * vocab + label among all (point, label) keys
    dev = g.device
    V = C5["vocab"]
    offs = torch.from_numpy(ls.offsets.astype(np.int64)).to(dev)
    labs = torch.from_numpy(ls.labels.astype(np.int64)).to(dev)
    owner = torch.repeat_interleave(torch.arange(n, device=dev), offs[1:] - offs[:-1])
    keys = torch.sort(owner * V + labs).values
    col = torch.arange(C5["R"], device=dev)[None, :]
    live = col < d[:, None]
    shared = torch.zeros_like(live)
    cnt = offs[1:] - offs[:-1]
    for j in range(int(cnt.max())):  # j-th label of each row
        has = (cnt > j)[:, None] & live
        lab = labs[torch.clamp(offs[:-1] + j, max=labs.numel() - 1)][:, None]
        q = torch.where(has, g * V + lab, torch.full_like(g, -1))
        pos = torch.clamp(torch.searchsorted(keys, q), max=keys.numel() - 1)
        shared |= has & (keys[pos] == q)
    bad = int((live & ~shared).sum())
    print(f"[c5f_1m] edges {int(live.sum())}, without a shared label {bad}", flush=True)
    assert bad == 0


# ----------------------------------------------------------------- stitched

def test_c5_stitched_equals_oracle():
    fx = FIX["c5s_1m"]
    n = fx["n"]
    x = D.synth_u8(42, 0, n, C5["dim"], C5["centers"], C5["sigma"])
    part = np.random.default_rng(44).integers(0, C5["parts"], n).astype(np.uint32)
    assert digest(x, part) == fx["input"]
    # label postings: points of each partition in ascending order
    pts = np.argsort(part, kind="stable").astype(np.uint32)
    off = np.zeros(C5["parts"] + 1, np.uint32)
    off[1:] = np.cumsum(np.bincount(part, minlength=C5["parts"]))
    graph, deg, medoids, st = D.stitched_build(x, off, pts, C5["Rsmall"], C5["Lsmall"], C5["Cs"], C5["STEPS"],
                                               C5["Rstitched"], row_cap=C5["Rstitched"])
    print(f"[c5s_1m] degree sum {int(deg.sum())} (oracle {fx['degree_sum']}), builds {st['build_sum_seconds']:.2f} s",
          flush=True)
    assert int(deg.sum()) == fx["degree_sum"]
    assert digest(graph, deg, medoids) == fx["graph"]
