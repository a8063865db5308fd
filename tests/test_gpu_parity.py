"""GPU parity: every HIP stage of the standard build against the CPU oracle,
bit for bit, on identical inputs (gfx950 only).

Each test feeds the HIP kernel (through the C ABI) and the oracle the same
seeded input and requires identical outputs: integer ids/degrees exactly and
fp32 distances bitwise (both sides implement the canonical distance order).
"""
import numpy as np
import pytest

import dance_amd as D
from oracle import oracle as O

pytestmark = pytest.mark.gpu

INV = 0xFFFFFFFF
FMAX = np.finfo(np.float32).max


def make_data(kind, n, dim, seed=7):
    rng = np.random.default_rng(seed)
    if kind == "f32":
        x = rng.standard_normal((n, dim)).astype(np.float32)
        return x / np.linalg.norm(x, axis=1, keepdims=True).astype(np.float32)
    if kind == "f16":
        return rng.standard_normal((n, dim)).astype(np.float16)
    return rng.integers(0, 256, (n, dim), dtype=np.uint8)


def random_work_state(data, R, C, seed, flt_max_noise=True):
    """Candidate rows with invalid ids, self loops, duplicates and (optionally)
    FLT_MAX distances. Without the noise every stored distance is the canonical
    distance of the row's vertex to the entry, as in every production work row
    (the reverse merge relies on it)."""
    rng = np.random.default_rng(seed)
    N = data.shape[0]
    s = O.State.empty(N, R, C)
    ids = rng.integers(0, N, (N, C)).astype(np.uint32)
    ids[rng.random((N, C)) < 0.08] = INV
    selfm = rng.random((N, C)) < 0.02
    ids[selfm] = np.broadcast_to(np.arange(N, dtype=np.uint32)[:, None], (N, C))[selfm]
    dupm = rng.random((N, C - 1)) < 0.06
    ids[:, 1:][dupm] = ids[:, :-1][dupm]
    a = np.repeat(np.arange(N, dtype=np.uint32), C)
    b = ids.ravel()
    ok = b < N
    d = np.full(N * C, FMAX, np.float32)
    d[ok] = O.distances(data, a[ok], b[ok])
    d = d.reshape(N, C)
    if flt_max_noise:
        d[rng.random((N, C)) < 0.01] = FMAX
    s.work = ids
    s.wd = d
    s.deg_work = rng.integers(0, C + 1, N).astype(np.uint32)
    return s


def to_dance(s):
    return D.GraphState(s.cur.copy(), s.deg_cur.copy(), s.work.copy(), s.deg_work.copy(), s.wd.copy())


def assert_state_equal(g, s, fields=("cur", "deg_cur", "work", "deg_work", "wd")):
    for f in fields:
        a, b = getattr(g, f), getattr(s, f)
        if f == "wd":
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{f} differs at {np.argwhere(a.view(np.uint32) != b.view(np.uint32))[:5]}"
        else:
            assert np.array_equal(a, b), f"{f} differs at {np.argwhere(a != b)[:5]}"


@pytest.mark.parametrize("kind,dim", [("f32", 96), ("f32", 100), ("f32", 7), ("u8", 128), ("u8", 192),
                                      ("u8", 33), ("f16", 96), ("f16", 50), ("f16", 97), ("f16", 33),
                                      ("f16", 1), ("f16", 255),
                                      # the widest rows of each type (16 chunks per lane)
                                      ("f32", 512), ("u8", 2048), ("f16", 1024), ("f32", 260)])
def test_distances_bitwise(kind, dim):
    data = make_data(kind, 3000, dim, seed=dim)
    rng = np.random.default_rng(1)
    a = rng.integers(0, 3000, 20000).astype(np.uint32)
    b = rng.integers(0, 3000, 20000).astype(np.uint32)
    g = D.stage_distances(data, a, b)
    o = O.distances(data, a, b)
    assert np.array_equal(g.view(np.uint32), o.view(np.uint32))


@pytest.mark.parametrize("dim", [96, 97, 8, 3])
def test_distances_f16_binary16_edges(dim):
    """fp16 rows whose binary16 differences round, go subnormal or overflow
    the square to inf (|a - b| > 256), and odd tails squared in fp32."""
    rng = np.random.default_rng(dim)
    n = 512
    x = (rng.standard_normal((n, dim)) * 10.0 ** rng.integers(-6, 3, (n, 1))).astype(np.float16)
    x[::7, 0] = np.float16(300.0)
    x[1::7, -1] = np.float16(-300.0)
    a = rng.integers(0, n, 8000).astype(np.uint32)
    b = rng.integers(0, n, 8000).astype(np.uint32)
    g = D.stage_distances(x, a, b)
    o = O.distances(x, a, b)
    assert np.isinf(o).any() and np.isfinite(o).any()
    assert np.array_equal(g.view(np.uint32), o.view(np.uint32))


@pytest.mark.parametrize("kind,n", [("f32", 5000), ("u8", 3000), ("f32", 700), ("f32", 1)])
def test_medoid(kind, n):
    data = make_data(kind, n, 96 if kind == "f32" else 128)
    gm, gs, gc = D.stage_medoid(data)
    om, os_, oc = O.medoid(data)
    assert np.array_equal(gc, oc)
    assert np.array_equal(gs.view(np.uint32), os_.view(np.uint32))
    assert gm == om


@pytest.mark.parametrize("kind,R,C", [("f32", 64, 80), ("u8", 32, 48), ("f32", 100, 130)])
def test_init(kind, R, C):
    data = make_data(kind, 2000, 96 if kind == "f32" else 128)
    g = D.stage_init(data, R, C)
    s = O.init_graph(data, R, C)
    assert_state_equal(g, s)


@pytest.mark.parametrize("kind", ["f32", "u8", "f16"])
@pytest.mark.parametrize("alpha,min_degree", [(1.0, 0), (1.2, 0), (1.2, 64), (1.2, 24)])
def test_prune_bitexact(kind, alpha, min_degree):
    dim = {"f32": 96, "u8": 128, "f16": 96}[kind]
    data = make_data(kind, 2500, dim, seed=3)
    R, C = 32, 80
    s0 = random_work_state(data, R, C, seed=11)
    g = D.stage_prune(data, to_dance(s0), min_degree, alpha)
    s = O.prune(data, s0, min_degree, alpha)
    assert_state_equal(g, s)


@pytest.mark.parametrize("kind", ["f32", "f16"])
@pytest.mark.parametrize("R,C", [(64, 200), (64, 64), (72, 100), (8, 256)])
def test_prune_shapes_bitexact(kind, R, C):
    """Wider and narrower rows than the build configurations (R up to 72, C up
    to 256, C = R), with the bound on for f32 / f16."""
    data = make_data(kind, 1500, 96, seed=4)
    s0 = random_work_state(data, R, C, seed=12)
    for alpha, md in ((1.0, 0), (1.2, 64)):
        g = D.stage_prune(data, to_dance(s0), md, alpha)
        s = O.prune(data, s0, md, alpha)
        assert_state_equal(g, s)


@pytest.mark.parametrize("rank,qbound", [("0", "1"), ("1", "0"), ("1", "1"), ("0", "0")])
@pytest.mark.parametrize("R,C", [(64, 80), (32, 128), (64, 64), (16, 100)])
def test_prune_kernels_bitexact(monkeypatch, rank, qbound, R, C):
    """Both prune kernels (k_prune; k_prune_rank for rows of at most 128
    candidates, with and without the bound's MFMA pair decisions) against
    the oracle, on rows with invalid ids, self loops, repeated ids and
    FLT_MAX distances."""
    monkeypatch.setenv("DANCE_PRUNE_RANK_ITERS", "0xF" if rank == "1" else "0x0")
    monkeypatch.setenv("DANCE_QBOUND", qbound)
    data = make_data("f32", 3000, 96, seed=R + C)
    s0 = random_work_state(data, R, C, seed=C)
    for alpha, md in ((1.0, 0), (1.2, 64), (1.2, 0)):
        g = D.stage_prune(data, to_dance(s0), md, alpha)
        s = O.prune(data, s0, md, alpha)
        assert_state_equal(g, s)


@pytest.mark.parametrize("gram", ["1", "0"])
@pytest.mark.parametrize("dim,levels", [(128, 256), (33, 256), (192, 256), (512, 256), (2048, 256), (128, 3)])
@pytest.mark.parametrize("R,C", [(64, 80), (32, 128), (16, 100)])
def test_prune_rank_u8_bitexact(monkeypatch, gram, dim, levels, R, C):
    """k_prune_rank on uint8 rows, with every pair's distance from int8 MFMA
    Gram tiles (gram 1) or tested inside the rounds (gram 0), against the
    oracle: rows of 1, 2, 4 and 16 chunks per lane, a width that is not a
    multiple of 32 bytes, rows of up to 128 candidates (four tiles), distances
    above 2^24 (rounded to float), and three-level data (many equal
    distances), on rows with invalid ids, self loops, repeated ids and FLT_MAX
    distances."""
    monkeypatch.setenv("DANCE_PRUNE_RANK_ITERS", "0xF")
    monkeypatch.setenv("DANCE_PRUNE_GRAM", gram)
    n = 1500 if dim <= 512 else 300
    rng = np.random.default_rng(dim + levels + C)
    data = rng.integers(0, levels, (n, dim)).astype(np.uint8)
    if levels == 3:
        data *= 100  # values 0, 100, 200
    s0 = random_work_state(data, R, C, seed=C + dim)
    for alpha, md in ((1.0, 0), (1.2, 64), (1.2, 0)):
        g = D.stage_prune(data, to_dance(s0), md, alpha)
        s = O.prune(data, s0, md, alpha)
        assert_state_equal(g, s)


@pytest.mark.parametrize("kind", ["f32", "u8"])
@pytest.mark.parametrize("heavy", [(0, 0), (8, 12)])
def test_reverse_merge_bitexact(kind, heavy):
    dim = 96 if kind == "f32" else 128
    data = make_data(kind, 3000, dim, seed=5)
    R, C = 32, 48
    s0 = random_work_state(data, R, C, seed=21, flt_max_noise=False)
    g, goff, gids = D.stage_reverse_merge(data, to_dance(s0), *heavy)
    s, ooff, oids = O.reverse_merge(data, s0, *heavy)
    assert np.array_equal(goff, ooff)
    assert np.array_equal(gids, oids)
    assert_state_equal(g, s, ("work", "deg_work", "wd"))


@pytest.mark.parametrize("cap", [32 * 1000, 32 * 300 + 5, 32 * 2999])
def test_reverse_merge_split_sort(monkeypatch, cap):
    """The reverse CSR sorted in parts of at most `cap` slots (the path of
    graphs with 2^32 or more slots, forced small): offsets, sources and the
    merged rows equal the oracle's (3, 10 and 2 parts; the last part short)."""
    monkeypatch.setenv("DANCE_REVERSE_PART_ITEMS", str(cap))
    data = make_data("f32", 3000, 96, seed=5)
    R, C = 32, 48
    s0 = random_work_state(data, R, C, seed=22, flt_max_noise=False)
    for heavy in ((0, 0), (8, 12)):
        g, goff, gids = D.stage_reverse_merge(data, to_dance(s0), *heavy)
        s, ooff, oids = O.reverse_merge(data, s0, *heavy)
        assert np.array_equal(goff, ooff)
        assert np.array_equal(gids, oids)
        assert_state_equal(g, s, ("work", "deg_work", "wd"))


def test_end_to_end_split_reverse_sort(monkeypatch):
    """The whole build with the reverse sort in parts equals the oracle."""
    monkeypatch.setenv("DANCE_REVERSE_PART_ITEMS", str(64 * 1237))
    data = make_data("f32", 4000, 96, seed=29)
    res = D.vamana_build(data, 64, 100, 80, 64)
    og, od, om = O.vnew2_build(data, 64, 100, 80, 64)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)


@pytest.mark.parametrize("kind,R,L,C,steps", [("f32", 32, 64, 48, 32), ("f32", 64, 100, 80, 64),
                                              ("u8", 32, 64, 48, 48), ("f32", 16, 150, 40, 100)])
def test_search_bitexact(kind, R, L, C, steps):
    dim = 96 if kind == "f32" else 128
    data = make_data(kind, 3000, dim, seed=9)
    s0 = O.init_graph(data, R, C)
    start, _, _ = O.medoid(data)
    for alpha in (1.0, 1.2):
        g = D.stage_search(data, to_dance(s0), L, steps, alpha, start)
        s = O.search(data, s0, L, steps, alpha, start)
        assert_state_equal(g, s, ("work", "deg_work", "wd"))


def test_search_after_iterations():
    """Search on a pruned (dup-free, converged) graph, not only the random init."""
    data = make_data("f32", 3000, 96, seed=13)
    R, L, C, steps = 32, 64, 48, 48
    start, _, _ = O.medoid(data)
    s = O.init_graph(data, R, C)
    for it in range(2):
        s = O.search(data, s, L, steps, 1.0, start)
        s, _, _ = O.reverse_merge(data, s)
        s = O.prune(data, s, 0, 1.0)
    g = D.stage_search(data, to_dance(s), L, steps, 1.2, start)
    o = O.search(data, s, L, steps, 1.2, start)
    assert_state_equal(g, o, ("work", "deg_work", "wd"))


@pytest.mark.parametrize("kind,n,R,L,C,steps", [("f32", 3000, 32, 64, 48, 32), ("u8", 3000, 32, 64, 48, 32),
                                                ("f32", 4000, 64, 100, 80, 64)])
def test_end_to_end_graph_identical(kind, n, R, L, C, steps):
    dim = 96 if kind == "f32" else 128
    data = make_data(kind, n, dim, seed=17)
    res = D.vamana_build(data, R, L, C, steps)
    og, od, om = O.vnew2_build(data, R, L, C, steps)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)


@pytest.mark.parametrize("rank_iters", ["0x0", "0xF", "0x5"])
def test_end_to_end_prune_kernel_choice(rank_iters, monkeypatch):
    """The whole build with each prune kernel in every iteration, and mixed."""
    monkeypatch.setenv("DANCE_PRUNE_RANK_ITERS", rank_iters)
    data = make_data("f32", 5000, 96, seed=23)
    res = D.vamana_build(data, 64, 100, 80, 64)
    og, od, om = O.vnew2_build(data, 64, 100, 80, 64)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)


@pytest.mark.parametrize("alpha_from", [0, 2])
def test_end_to_end_alpha_schedule(alpha_from, monkeypatch):
    """The reference's alpha-schedule knobs (USE_ALPHA_FROM_FIRST_ITER = from
    0, VAMANA_ALPHA_FINAL_FROM_ITER = k) through DANCE_ALPHA_FROM_ITER."""
    monkeypatch.setenv("DANCE_ALPHA_FROM_ITER", str(alpha_from))
    data = make_data("f32", 4000, 96, seed=21)
    res = D.vamana_build(data, 32, 64, 48, 32)
    og, od, om = O.vnew2_build(data, 32, 64, 48, 32, alpha_from=alpha_from)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)
    default, _, _ = O.vnew2_build(data, 32, 64, 48, 32)
    assert not np.array_equal(default, og)  # the schedule changes the graph


@pytest.mark.parametrize("kind", ["f32", "u8"])
def test_end_to_end_locality_schedule(kind, monkeypatch):
    """The processing order never changes the graph: vertices sorted by their
    three nearest of K pivots (K = 1024 and K = 37), by the nearest alone
    (K = 2000, past the three-level key's range), or in id order (K = 0)."""
    data = make_data(kind, 4000, 96 if kind == "f32" else 64, seed=23)
    og, od, om = O.vnew2_build(data, 32, 64, 48, 32)
    runs = [("1024", None), ("37", None), ("2000", None), ("0", None)]
    if kind == "f32":
        runs.append(("1024", "0"))  # no code rows: the pivots from the fp32 rows (k_cells)
    for cells, qbound in runs:
        monkeypatch.setenv("DANCE_LOCALITY_CELLS", cells)
        if qbound is not None:
            monkeypatch.setenv("DANCE_QBOUND", qbound)
        res = D.vamana_build(data, 32, 64, 48, 32)
        assert res.medoid == om, cells
        assert np.array_equal(res.degree, od), cells
        assert np.array_equal(res.graph, og), cells


@pytest.mark.parametrize("kind,L,steps", [("f32", 300, 64), ("u8", 500, 80), ("f32", 1000, 100),
                                          ("f32", 257, 257), ("f32", 200, 64), ("u8", 160, 96),
                                          ("f32", 129, 64)])
def test_end_to_end_wide_search_list(kind, L, steps):
    """Build lists above 128 entries: the 4-slot pool (L 129-256, with the
    bound for fp32 rows and the random initial graph from k_init) and the
    16-slot pool above 256 (DiskANN callers build with L of several hundred
    and the reference sizes its pool by L, vnew2.cu:193-199, 2221), against
    the oracle."""
    dim = 96 if kind != "u8" else 128
    data = make_data(kind, 3000, dim, seed=L)
    res = D.vamana_build(data, 32, L, 48, steps)
    og, od, om = O.vnew2_build(data, 32, L, 48, steps)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)


@pytest.mark.parametrize("kind,iters,alpha_from", [("f32", 5, None), ("f32", 6, None), ("f32", 6, 0),
                                                    ("u8", 6, None), ("f32", 1, None), ("f32", 8, 5),
                                                    ("u8", 1, None), ("f32", 2, None), ("u8", 2, 0)])
def test_end_to_end_iteration_count(kind, iters, alpha_from, monkeypatch):
    """The reference's VAMANA_ITERS (gpu_vamana_config.h:78-79) through
    DANCE_VAMANA_ITERS, alone and with the alpha schedule knob; the kernel
    profile reports one launch per iteration."""
    monkeypatch.setenv("DANCE_VAMANA_ITERS", str(iters))
    if alpha_from is not None:
        monkeypatch.setenv("DANCE_ALPHA_FROM_ITER", str(alpha_from))
    dim = 96 if kind == "f32" else 128
    data = make_data(kind, 4000, dim, seed=29 + iters)
    res = D.vamana_build(data, 32, 64, 48, 32)
    og, od, om = O.vnew2_build(data, 32, 64, 48, 32, iters=iters, alpha_from=alpha_from)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)
    kp = D.last_kernel_profile()
    assert kp["iterations"] == iters and len(kp["search_iter_ms"]) == iters
    assert all(t > 0 for t in kp["search_iter_ms"]) and all(t > 0 for t in kp["prune_iter_ms"])


@pytest.mark.parametrize("kind,R,L,C,steps", [("f32", 96, 128, 128, 64), ("u8", 80, 100, 120, 48),
                                              ("f32", 72, 100, 250, 64)])
def test_end_to_end_wide_degree(kind, R, L, C, steps):
    # degrees above one 64-lane batch: the first iteration's recomputed
    # neighbours and every later gather take two batches; C = 128 is the
    # largest work row of the insert bound's variant, C = 250 runs without it
    data = make_data(kind, 3000, 96 if kind == "f32" else 128, seed=R)
    res = D.vamana_build(data, R, L, C, steps)
    og, od, om = O.vnew2_build(data, R, L, C, steps)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)


@pytest.mark.parametrize("kind", ["f32", "u8"])
@pytest.mark.parametrize("n", [1, 2, 3, 17, 130])
def test_end_to_end_tiny_inputs(kind, n):
    # one point (no neighbours), two, three, and rows shorter than R
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((n, 24)).astype(np.float32) if kind == "f32"
         else rng.integers(0, 256, (n, 32), dtype=np.uint8))
    res = D.vamana_build(x, 16, 24, 20, 12)
    og, od, om = O.vnew2_build(x, 16, 24, 20, 12)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)


@pytest.mark.parametrize("kind", ["f32", "u8"])
def test_end_to_end_duplicate_rows(kind):
    # 600 rows drawn from 12 distinct vectors: every search, insert and prune
    # decision is a tie at distance 0 or between equal distances, resolved by
    # slot and id order alone
    rng = np.random.default_rng(5)
    base = (rng.standard_normal((12, 24)).astype(np.float32) if kind == "f32"
            else rng.integers(0, 256, (12, 32), dtype=np.uint8))
    x = np.ascontiguousarray(base[rng.integers(0, 12, 600)])
    res = D.vamana_build(x, 16, 32, 24, 16)
    og, od, om = O.vnew2_build(x, 16, 32, 24, 16)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)


@pytest.mark.parametrize("kind,dim", [("f32", 512), ("u8", 2048), ("f32", 200)])
def test_end_to_end_wide_rows(kind, dim):
    # the widest supported rows (16 chunks of 16 bytes per lane) and a width
    # whose last chunk group is partial
    data = make_data(kind, 1500, dim, seed=dim)
    res = D.vamana_build(data, 32, 48, 40, 24)
    og, od, om = O.vnew2_build(data, 32, 48, 40, 24)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)


def test_sort_pairs_and_scan():
    rng = np.random.default_rng(3)
    for n, bits in [(1, 8), (4095, 12), (4097, 17), (300000, 20), (70000, 24)]:
        keys = rng.integers(0, 1 << bits, n).astype(np.uint32)
        vals = np.arange(n, dtype=np.uint32)
        ok, ov = D.stage_sort_pairs(keys, vals, bits)
        order = np.argsort(keys, kind="stable")
        assert np.array_equal(ok, keys[order])
        assert np.array_equal(ov, vals[order])
    for n in (1, 4096, 4097, 5_000_000):
        x = rng.integers(0, 100, n).astype(np.uint32)
        ex = np.concatenate([[0], np.cumsum(x, dtype=np.uint64)[:-1]]).astype(np.uint32)
        assert np.array_equal(D.stage_scan(x), ex)


def test_fast_small_profile_fp16_storage():
    """FAST_SMALL stores float input as fp16 (round to nearest even) and builds
    on it; the graph equals the oracle's build on the same fp16 rows."""
    data = make_data("f32", 3000, 96, seed=23)
    try:
        D.set_profile("FAST_SMALL")
        res = D.vamana_build(data, 32, 64, 48, 32)
    finally:
        D.set_profile("QUALITY")
    og, od, om = O.vnew2_build(data.astype(np.float16), 32, 64, 48, 32)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)


def test_build_device_handoff():
    """gpu_vamana_vnew2_build_device_float keeps data/graph/degree on the device
    and hands ownership to the caller (hipFree)."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipFree.argtypes = [C.c_void_p]
    data = make_data("f32", 2000, 96, seed=29)
    N, R = 2000, 32
    dd, dg, ddeg = C.c_void_p(), C.c_void_p(), C.c_void_p()
    rc = D.lib().gpu_vamana_vnew2_build_device_float(data.ctypes.data, N, 96, R, 64, 48, 32, C.byref(dd),
                                                     C.byref(dg), C.byref(ddeg))
    assert rc == 0 and dd.value and dg.value and ddeg.value
    back = np.empty_like(data)
    graph = np.empty((N, R), np.uint32)
    deg = np.empty(N, np.uint32)
    assert hip.hipMemcpy(back.ctypes.data, dd, back.nbytes, 2) == 0
    assert hip.hipMemcpy(graph.ctypes.data, dg, graph.nbytes, 2) == 0
    assert hip.hipMemcpy(deg.ctypes.data, ddeg, deg.nbytes, 2) == 0
    for p in (dd, dg, ddeg):
        assert hip.hipFree(p) == 0
    assert np.array_equal(back, data)
    og, od, om = O.vnew2_build(data, R, 64, 48, 32)
    assert np.array_equal(graph, og) and np.array_equal(deg, od)
    assert D.lib().gpu_vamana_vnew2_get_last_medoid() == om
