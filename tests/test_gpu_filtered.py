"""GPU parity of the label-filtered build ("canonical_v2",
/root/reference/src/gpu_vamana_filtered.cu:5663-6483) against the CPU oracle:
identical seeded inputs, identical graphs (ids, order, degrees) and identical
diagnostics, after 0 (random backbone), 1 and 3 rounds."""
import numpy as np
import pytest

from dance_amd import INVALID
from dance_amd import filtered as F
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def make_case(kind, n, dim, vocab, max_per, seed, hub=False):
    rng = np.random.default_rng(seed)
    if kind == "u8":
        x = rng.integers(0, 256, (n, dim), dtype=np.uint8)
    else:
        centers = rng.standard_normal((16, dim)).astype(np.float32)
        x = centers[rng.integers(0, 16, n)] + 0.4 * rng.standard_normal((n, dim)).astype(np.float32)
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        if kind == "f16":
            x = x.astype(np.float16)
    ls = F.synth_labels(n, vocab, 1, max_per, 1.0, seed=seed + 1)
    if hub:
        # a point at the origin carrying the ten most frequent labels is the
        # nearest neighbour of every unit vector: its reverse list is long
        x[0] = 0
        rows = [list(range(10))] + [list(ls.row(i)) for i in range(1, n)]
        ls = F.canonical_labels(rows, vocab)
    return x, ls


def oracle_rows(x):
    return x.astype(np.float16) if x.dtype == np.float32 else x


def run_both(x, ls, starts, gstart, R, L, FL, C_, steps, alpha=1.2, universal=INVALID, rounds=3, publish_R=0):
    """publish_R: the DISKANN_GPU_FILTERED_PUBLISH_DEGREE the caller set (0: none)."""
    res_rc = F.build_rc(x, ls, starts, R, L, FL, C_, steps, alpha, universal, gstart, rounds,
                        graph=(g := np.empty((x.shape[0], R), np.uint32)), degree=(d := np.empty(x.shape[0], np.uint32)))
    if 0 < publish_R < R:
        g = g.ravel()[:x.shape[0] * publish_R].reshape(x.shape[0], publish_R)
    orc, og, od, diag = O.filtered_build(oracle_rows(x), ls.offsets, ls.labels, starts, ls.num_labels, R, L, FL, C_,
                                         steps, alpha, universal, gstart, rounds, publish_R)
    return res_rc, g, d, orc, og, od, diag


def assert_same(x, ls, starts, gstart, R, L, FL, C_, steps, **kw):
    rc, g, d, orc, og, od, diag = run_both(x, ls, starts, gstart, R, L, FL, C_, steps, **kw)
    assert rc == orc == 0
    assert np.array_equal(d, od), f"degree differs at rows {np.nonzero(d != od)[0][:8]}"
    bad = np.nonzero((g != og).any(1))[0]
    assert bad.size == 0, f"rows differ: {bad[:8]} gpu={g[bad[0]][:d[bad[0]]]} oracle={og[bad[0]][:od[bad[0]]]}"
    st = F.last_stats()
    assert st["invalid_neighbor_count"] == diag[0] and st["self_loop_count"] == diag[1]
    assert st["low_common_label_degree_count"] == diag[2]
    assert (st["out_degree_min"], st["out_degree_max"]) == (diag[3], diag[4])
    assert (st["common_label_degree_min"], st["common_label_degree_max"]) == (diag[5], diag[6])
    assert st["unfiltered_candidate_count"] == diag[7] and st["filtered_candidate_count"] == diag[8]
    assert (st["label_check_count"], st["label_reject_count"], st["universal_label_pass_count"]) == tuple(diag[9:12])
    assert st["semantic_stage"] == 6 and st["semantic_complete"] == 1
    return g, d, diag


@pytest.mark.parametrize("rounds", [0, 1, 3])
@pytest.mark.parametrize("kind", ["u8", "f32"])
def test_filtered_rounds_identical(kind, rounds):
    x, ls = make_case(kind, 3000, 64 if kind == "u8" else 96, 40, 4, seed=11)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    g, d, diag = assert_same(x, ls, starts, gs, 32, 64, 64, 750, 32, rounds=rounds)
    if rounds == 0:
        assert (d == 16).all()
    else:
        assert diag[0] == 0 and diag[1] == 0


def test_filtered_fp16_rows_extension_entry():
    x, ls = make_case("f16", 2500, 96, 30, 3, seed=5)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    assert_same(x, ls, starts, gs, 24, 48, 48, 64, 24, rounds=2)


@pytest.mark.parametrize("FL,C_,R,L", [(20, 64, 32, 64), (100, 750, 64, 100), (8, 128, 16, 12)])
def test_filtered_pool_and_capacity_edges(FL, C_, R, L):
    """Pools below 32/64 (filtered_L), work capacity exactly 2R, L < R."""
    x, ls = make_case("u8", 2000, 64, 25, 5, seed=FL + C_)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    assert_same(x, ls, starts, gs, R, L, FL, C_, 24)


def test_filtered_universal_label_and_missing_starts():
    """Universal label (never a task; matches everything in diagnostics),
    labels >= num_labels (no postings), unlabelled rows, invalid starts and
    an invalid global start."""
    x, ls = make_case("u8", 2500, 64, 30, 4, seed=9)
    rows = [list(ls.row(i)) for i in range(2500)]
    for i in range(0, 2500, 7):
        rows[i] = rows[i] + [0]          # label 0 = universal on every 7th row
    for i in range(3, 2500, 11):
        rows[i] = []                     # unlabelled
    for i in range(5, 2500, 13):
        rows[i] = rows[i] + [31, 33]     # beyond num_labels = 30
    ls = F.canonical_labels(rows, 30)
    starts = F.label_starts(x, ls)
    starts[[2, 5, 17]] = INVALID
    starts[4] = 10 ** 6                  # out of range: skipped like INVALID
    assert_same(x, ls, starts, INVALID, 32, 64, 64, 750, 32, universal=0)
    assert_same(x, ls, starts, F.global_start(x), 32, 64, 64, 750, 32, universal=0, rounds=1)


def test_filtered_wide_label_rows():
    """Rows with 9-12 labels and rows carrying the label 0xFFFFFFFF mixed with
    ordinary rows: membership tests read the fixed-width label table where a
    point's list fits it and walk the list otherwise."""
    x, ls = make_case("u8", 2500, 64, 40, 4, seed=21)
    rng = np.random.default_rng(22)
    rows = [list(ls.row(i)) for i in range(2500)]
    for i in range(0, 2500, 5):
        rows[i] = sorted(set(rows[i]) | set(int(v) for v in rng.choice(40, int(rng.integers(9, 13)), replace=False)))
    for i in range(3, 2500, 17):
        rows[i] = rows[i] + [0xFFFFFFFF]
    ls = F.canonical_labels(rows, 40)
    starts = F.label_starts(x, ls)
    assert_same(x, ls, starts, F.global_start(x), 32, 64, 64, 750, 32)


def test_filtered_hub_long_reverse_lists():
    """A hub with in-degree far above 256 takes the global-memory prune path."""
    x, ls = make_case("f32", 3000, 64, 40, 3, seed=21, hub=True)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    g, d, _ = assert_same(x, ls, starts, gs, 32, 64, 64, 750, 32, rounds=1)
    assert F.last_profile()["long_lists"] > 0


@pytest.mark.parametrize("alpha", [0.5, 1.2, 3.0])
def test_filtered_hub_long_prune(alpha):
    """Long lists are pruned by one workgroup per row (selection reduced over
    the waves); alpha 0.5 occludes so much that selections reach deep into
    the list. A block of identical vectors gives tied distances and zero pair
    distances."""
    x, ls = make_case("f32", 3000, 64, 40, 3, seed=25, hub=True)
    x[100:400] = x[100]
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    assert_same(x, ls, starts, gs, 32, 64, 64, 750, 32, alpha=alpha, rounds=1)
    p = F.last_profile()
    assert p["long_lists"] > 0 and p["long_max_candidates"] > 256


def test_filtered_hub_deep_selection():
    """One shared label makes every pair coverable, so alpha 0.5 occludes
    about half the sphere per selection: the hub's selections run past its
    256 nearest candidates."""
    rng = np.random.default_rng(27)
    x = rng.standard_normal((3000, 64)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    x[0] = 0  # distance 1 to every other point, which are ~2 apart: everyone's first pick
    ls = F.canonical_labels([[0]] * 3000, 1)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    assert_same(x, ls, starts, gs, 32, 64, 64, 750, 32, alpha=0.5, rounds=1)
    p = F.last_profile()
    assert p["long_lists"] > 0
    assert p["long_max_candidates"] > 2048  # the hub's entries wrap around the workgroup's 16 waves


@pytest.mark.parametrize("alpha", [0.5, 1.2])
def test_filtered_hub_key_windows(alpha):
    """A hub whose candidate list (distances spread by radius) is longer than
    the long prune's key window (2048): the prune walks several windows,
    replaying earlier selections on each."""
    rng = np.random.default_rng(31)
    n = 20000
    x = rng.standard_normal((n, 32)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    x *= rng.uniform(1.0, 3.0, (n, 1)).astype(np.float32)
    x[0] = 0  # every point's nearest neighbour
    ls = F.canonical_labels([[0]] * n, 1)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    assert_same(x, ls, starts, gs, 32, 64, 64, 750, 32, alpha=alpha, rounds=1)
    p = F.last_profile()
    assert p["long_max_candidates"] > 2 * 2048


@pytest.mark.parametrize("alpha", [0.5, 1.2])
def test_filtered_hub_tied_keys(alpha):
    """Every candidate of the hub lies at the same distance (u8 rows with
    exactly eight ones around an all-zero hub): one key window holds more
    entries than its LDS list (4096), so the prune scans the list with the
    window's key filter instead."""
    rng = np.random.default_rng(33)
    n = 6000
    x = np.zeros((n, 64), np.uint8)
    for i in range(1, n):
        x[i, rng.choice(64, 8, replace=False)] = 1
    ls = F.canonical_labels([[0]] * n, 1)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    assert_same(x, ls, starts, gs, 32, 64, 64, 750, 32, alpha=alpha, rounds=1)
    p = F.last_profile()
    assert p["long_max_candidates"] > 4096


@pytest.mark.parametrize("n", [1, 2, 17, 50])
def test_filtered_tiny(n):
    x, ls = make_case("u8", n, 32, 5, 3, seed=n)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    assert_same(x, ls, starts, gs, 16, 32, 32, 64, 16)


@pytest.mark.parametrize("kind", ["u8", "f32"])
def test_filtered_duplicate_rows(kind):
    """1500 rows drawn from 10 distinct vectors: the canonical pools, the
    merge and FilteredRobustPrune meet equal distances everywhere and order
    them by id alone."""
    x, ls = make_case(kind, 1500, 32, 12, 3, seed=23)
    rng = np.random.default_rng(3)
    x = np.ascontiguousarray(x[rng.integers(0, 10, 1500)])
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    assert_same(x, ls, starts, gs, 16, 32, 32, 64, 16)


def log_fields(line):
    return dict(tok.split("=", 1) for tok in line.split()[1:])


def degree_profile(g, d, ls, universal):
    """canonical_print_round_diagnostics (gpu_vamana_filtered.cu:94-160)
    restated over the returned graph: entry floor(q * (N - 1)) of the sorted
    degrees, label-compatible degrees and per-label minimum degrees."""
    N, R = g.shape
    sets = [set(ls.row(i).tolist()) for i in range(N)]
    deg = np.minimum(d, R)
    compat, minpl = np.zeros(N, np.int64), np.zeros(N, np.int64)
    for r in range(N):
        nb = [int(v) for v in g[r, :deg[r]] if v < N]
        labs = ls.row(r).tolist()
        compat[r] = sum(1 for v in nb if any(lab == universal or lab in sets[v] for lab in labs))
        spec = [lab for lab in labs if lab != universal]
        minpl[r] = min(sum(1 for v in nb if lab in sets[v]) for lab in spec) if spec else compat[r]

    def pct(v, q):
        return int(np.sort(v)[int(q * (N - 1))])
    out = {"avg": f"{deg.sum() / N:.3f}", "degree_eq_R_frac": f"{(deg == R).sum() / N:.6f}",
           "compatible_avg": f"{compat.sum() / N:.3f}", "min_per_label_avg": f"{minpl.sum() / N:.3f}"}
    for q, tag in ((0.50, "p50"), (0.95, "p95"), (0.99, "p99")):
        out[tag] = str(pct(d, q))
        out["compatible_" + tag] = str(pct(compat, q))
        out["min_per_label_" + tag] = str(pct(minpl, q))
    return out


@pytest.mark.parametrize("universal,PR", [(INVALID, 0), (0, 0), (INVALID, 24)])
def test_filtered_build_log(capfd, monkeypatch, universal, PR):
    """The reference-format build log (gpu_vamana_filtered.cu:5723-5730,
    :6294-6297, :6325, :94-160): the policy banner, one line per round whose
    changed / touched / reverse-proposal counts equal the oracle's, the
    coverage-repair line, and the degree percentiles of the published graph."""
    monkeypatch.setenv("DANCE_FILTERED_LOG", "1")
    if PR:
        monkeypatch.setenv("DISKANN_GPU_FILTERED_PUBLISH_DEGREE", str(PR))
    x, ls = make_case("u8", 2500, 64, 30, 4, seed=13)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    capfd.readouterr()
    g, d, _ = assert_same(x, ls, starts, gs, 32, 64, 48, 750, 32, universal=universal, rounds=3, publish_R=PR)
    want = O.filtered_round_log()
    lines = capfd.readouterr().out.splitlines()
    pol = [log_fields(s) for s in lines if s.startswith("[gpu_vamana_filtered_navigation_policy]")]
    assert len(pol) == 1
    assert pol[0] == {"per_label_pool": "32", "per_label_keep": "8", "true_ordinary_round0": "0",
                      "pure_ordinary_round0": "0", "ordinary_pool": "48", "ordinary_steps": "32",
                      "posting_anchor": "0", "additional_round0_anchor": "0", "bridge_work_reserve": "8",
                      "active_frontier": "0", "label_quota": "1", "exact_csr_reverse": "1"}
    rounds = [log_fields(s) for s in lines if s.startswith("[gpu_vamana_filtered_canonical_round]")]
    assert len(rounds) == 3
    N, T = x.shape[0], ls.labels.size
    for r, f in enumerate(rounds):
        assert f == {"round": str(r), "kind": "full", "alpha": "1.200", "active": str(N), "tasks": str(T),
                     "changed": str(want[r, 0]), "touched": str(want[r, 1]),
                     "reverse_proposals": str(want[r, 2]), "deficient": "0", "next_active": str(N)}
        assert 0 < want[r, 1] <= N and want[r, 2] >= want[r, 1]
    assert "[gpu_vamana_filtered_label_coverage_repair] disabled=1" in lines
    deg = [log_fields(s) for s in lines if s.startswith("[gpu_vamana_filtered_canonical_degree]")]
    assert len(deg) == 1
    secs = float(deg[0].pop("diagnostic_seconds"))
    assert secs >= 0
    assert deg[0] == degree_profile(g, d, ls, universal)


def test_filtered_abi_float_entry_equals_oracle():
    """gpu_vamana_filtered_build_float (the reference entry: float input is
    searched as round-to-nearest fp16 rows, filtered.cu:6497-6503) against
    the oracle's filtered build of the same rows; the extension entry on the
    rounded fp16 rows gives the same graph."""
    x, ls = make_case("f32", 2000, 96, 30, 3, seed=3)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    a = F.filtered_build(x, ls, starts, 32, 64, 64, 750, 32, 1.2, INVALID, gs)
    orc, og, od, _ = O.filtered_build(x, ls.offsets, ls.labels, starts, ls.num_labels, 32, 64, 64, 750, 32, 1.2,
                                      INVALID, gs, 3)
    assert orc == 0 and np.array_equal(a.graph, og) and np.array_equal(a.degree, od)
    b = F.filtered_build(x.astype(np.float16), ls, starts, 32, 64, 64, 750, 32, 1.2, INVALID, gs)
    assert np.array_equal(b.graph, og) and np.array_equal(b.degree, od)
    assert a.profile["rounds"] == 3 and a.stats["gpu_build_seconds"] > 0


@pytest.mark.parametrize("kind,PR,hub,rounds", [("u8", 8, False, 3), ("f32", 24, True, 3), ("u8", 40, False, 3),
                                                ("f32", 63, True, 3), ("u8", 16, False, 0)])
def test_filtered_publish_degree(monkeypatch, kind, PR, hub, rounds):
    # DISKANN_GPU_FILTERED_PUBLISH_DEGREE below R: the publish step
    # (gpu_vamana_filtered.cu:6328-6432) against the oracle's
    monkeypatch.setenv("DISKANN_GPU_FILTERED_PUBLISH_DEGREE", str(PR))
    x, ls = make_case(kind, 3000, 64 if kind == "u8" else 96, 40, 4, seed=17, hub=hub)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    g, d, diag = assert_same(x, ls, starts, gs, 64, 100, 100, 750, 64, rounds=rounds, publish_R=PR)
    assert g.shape == (3000, PR) and d.max() <= PR
    p = F.last_profile()
    assert p["publish_degree"] == PR and p["publish_touched"] > 0 and p["publish_ms"] > 0
    if hub:  # the hub (in-degree > 1000 after the forward pass) takes global scratch
        assert p["publish_long_entries"] > 1000
    res = F.filtered_build(x, ls, starts, R=64, L=100, filtered_L=100, STEPS=64, gstart=gs, rounds=rounds)
    assert res.graph.shape == (3000, PR) and np.array_equal(res.graph, g)


@pytest.mark.parametrize("value", ["64", "500", "0", "-3", "abc"])
def test_filtered_publish_degree_inactive(monkeypatch, value):
    # values at or above R, and non-positive ones, publish the build graph as is
    x, ls = make_case("u8", 1500, 32, 20, 3, seed=23)
    starts, gs = F.label_starts(x, ls), F.global_start(x)
    monkeypatch.delenv("DISKANN_GPU_FILTERED_PUBLISH_DEGREE", raising=False)
    base = F.filtered_build(x, ls, starts, R=64, L=64, filtered_L=64, STEPS=32, gstart=gs)
    monkeypatch.setenv("DISKANN_GPU_FILTERED_PUBLISH_DEGREE", value)
    res = F.filtered_build(x, ls, starts, R=64, L=64, filtered_L=64, STEPS=32, gstart=gs)
    assert res.profile["publish_degree"] == 64 and res.profile["publish_touched"] == 0
    assert np.array_equal(res.graph, base.graph) and np.array_equal(res.degree, base.degree)
