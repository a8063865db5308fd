"""The search's quantized distance bound (dance_amd/csrc/qbound.h).

The bound may only flag a pair when the canonical distance is >= the
threshold; it is probed right at the threshold (T = d and the next float
above d) on adversarial rows: exact and one-ulp duplicates, tiny, huge,
zero and integer-valued rows, non-finite rows. Builds and searches with the
bound off, on in the first iteration (default) and on in every iteration
must give the oracle's graph bit for bit.
"""
import os

import numpy as np
import pytest

import dance_amd as D
from oracle import oracle as O

pytestmark = pytest.mark.gpu

FMAX = np.finfo(np.float32).max


def adversarial(n, dim, seed, dtype=np.float32, huge=True):
    """huge=False keeps every value finite in fp16."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, dim))
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    x = x.astype(np.float32)
    x[10:20] = x[0]                                   # exact duplicates
    x[20:40] = x[1]
    x[20:40, 0] = np.nextafter(x[20:40, 0], np.float32(np.inf))  # one ulp apart
    x[40:50] *= np.float32(1e-20)                     # scale below the coded range
    x[50:60] *= np.float32(1e9 if huge else 300.0)    # large but coded
    x[60:70] *= np.float32(1e17 if huge else 3e4)     # scale above the coded range (fp32)
    x[70:80] = 0.0                                    # zero rows
    x[80:90] = rng.integers(-3, 4, (10, dim))         # exact small integers
    x[90:100] = x[91] + np.float32(1e-7) * rng.standard_normal((10, dim)).astype(np.float32)
    return x.astype(dtype)


def pairs(n, m, seed):
    rng = np.random.default_rng(seed)
    a = rng.integers(0, n, m).astype(np.uint32)
    b = rng.integers(0, n, m).astype(np.uint32)
    special = np.arange(0, 100, dtype=np.uint32)  # every adversarial row against its neighbours
    a = np.concatenate([a, special, special, np.zeros(100, np.uint32)])
    b = np.concatenate([b, (special + 1) % n, (special + 7) % n, special])
    return a, b


def check_sound(x, a, b):
    d = D.stage_distances(x, a, b)
    above = np.nextafter(d, np.float32(np.inf))
    flagged_any = 0
    for T in (d, above, d * np.float32(1 + 1e-6), d * np.float32(0.999), d * np.float32(0.5),
              np.zeros_like(d), np.full_like(d, FMAX), np.full_like(d, 1e-38)):
        T = np.ascontiguousarray(T, np.float32)
        f = D.stage_qbound(x, a, b, T).astype(bool)
        bad = f & ~(d >= T)
        assert not bad.any(), f"bound flagged dist < T at {np.nonzero(bad)[0][:5]}: d={d[bad][:3]} T={T[bad][:3]}"
        flagged_any += int(f.sum())
    assert not D.stage_qbound(x, a, b, above).any()  # no pair has dist >= next float above it
    return flagged_any


@pytest.mark.parametrize("dim", [96, 112, 20, 1, 7])
def test_bound_is_sound_f32(dim):
    x = adversarial(4000, dim, seed=dim)
    a, b = pairs(4000, 20000, seed=dim + 1)
    assert check_sound(x, a, b) > 0


def test_bound_is_sound_f16():
    x = adversarial(3000, 96, seed=5, dtype=np.float16, huge=False)
    a, b = pairs(3000, 20000, seed=6)
    assert check_sound(x, a, b) > 0


def check_insert_bound_sound(x, a, b, alpha):
    """Every pair the insert bound decides is decided as the exact test
    fl(alpha * dist) <= T0 would decide it, for T0 at, one ulp either side
    of, and well away from fl(alpha * dist), and for degenerate T0."""
    d = D.stage_distances(x, a, b)
    al = np.float32(alpha)
    ad = al * d  # fl(alpha * dist), as the insert evaluates it
    yes_total = no_total = 0
    with np.errstate(invalid="ignore", over="ignore"):
        for T0 in (ad, np.nextafter(ad, np.float32(-np.inf)), np.nextafter(ad, np.float32(np.inf)),
                   ad * np.float32(1.5), ad * np.float32(0.7), ad * np.float32(1 + 1e-6), ad * np.float32(1 - 1e-6),
                   np.zeros_like(d), np.full_like(d, FMAX), np.full_like(d, 1e-38), np.full_like(d, 1e30),
                   np.full_like(d, np.float32(np.nanmedian(ad[np.isfinite(ad)])))):
            T0 = np.ascontiguousarray(T0, np.float32)
            f = D.stage_insert_bound(x, a, b, T0, alpha)
            holds = ad <= T0
            bad_yes = (f == 1) & ~holds
            bad_no = (f == 2) & holds
            assert not bad_yes.any(), f"upper bound wrong at {np.nonzero(bad_yes)[0][:5]}: ad={ad[bad_yes][:3]} T0={T0[bad_yes][:3]}"
            assert not bad_no.any(), f"lower bound wrong at {np.nonzero(bad_no)[0][:5]}: ad={ad[bad_no][:3]} T0={T0[bad_no][:3]}"
            assert set(np.unique(f)) <= {0, 1, 2}
            yes_total += int((f == 1).sum())
            no_total += int((f == 2).sum())
    return yes_total, no_total


@pytest.mark.parametrize("alpha", [1.0, 1.2, 2.0, 0.8])
@pytest.mark.parametrize("dim", [96, 112, 20, 7])
def test_insert_bound_is_sound_f32(dim, alpha):
    x = adversarial(4000, dim, seed=dim + 3)
    a, b = pairs(4000, 20000, seed=dim + 4)
    yes, no = check_insert_bound_sound(x, a, b, alpha)
    assert yes > 0 and no > 0


@pytest.mark.parametrize("alpha", [1.0, 1.2])
def test_insert_bound_is_sound_f16(alpha):
    """fp16 rows up to 3e4 (binary16 squares overflow to +inf past a
    difference of 256): the upper bound's cap keeps it from proving those."""
    x = adversarial(3000, 96, seed=9, dtype=np.float16, huge=False)
    a, b = pairs(3000, 20000, seed=10)
    yes, no = check_insert_bound_sound(x, a, b, alpha)
    assert yes > 0 and no > 0
    big = np.arange(60, 70, dtype=np.uint32)  # rows scaled by 3e4
    aa = np.repeat(big, 3000)
    bb = np.tile(np.arange(3000, dtype=np.uint32), 10)
    d = D.stage_distances(x, aa, bb)
    assert np.isinf(d).any()
    f = D.stage_insert_bound(x, aa, bb, np.full(aa.shape[0], 1e30, np.float32), alpha)
    assert not (f[np.isinf(d)] == 1).any()


def test_insert_bound_never_decides_non_finite_rows_wrongly():
    x = adversarial(500, 96, seed=8)
    x[100] = np.inf
    x[101, 3] = np.nan
    x[102, 5] = -np.inf
    a = np.repeat(np.arange(100, 103, dtype=np.uint32), 500)
    b = np.tile(np.arange(500, dtype=np.uint32), 3)
    for aa, bb in ((a, b), (b, a)):
        for T0 in (np.full(aa.shape[0], FMAX, np.float32), np.full(aa.shape[0], 1.0, np.float32)):
            f = D.stage_insert_bound(x, aa, bb, T0, 1.2)
            assert not f.any()  # r = +inf rows: neither bound proves anything


def test_bound_never_flags_non_finite_rows():
    x = adversarial(500, 96, seed=8)
    x[100] = np.inf
    x[101, 3] = np.nan
    x[102, 5] = -np.inf
    a = np.repeat(np.arange(100, 103, dtype=np.uint32), 500)
    b = np.tile(np.arange(500, dtype=np.uint32), 3)
    for aa, bb in ((a, b), (b, a)):
        f = D.stage_qbound(x, aa, bb, np.zeros(aa.shape[0], np.float32))
        assert not f.any()


def test_bound_is_strong_on_far_pairs():
    """Far below the distance the bound proves almost every pair (the
    property the search relies on for its speed, not for its results)."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3000, 96)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    a, b = pairs(3000, 20000, seed=12)
    keep = a != b
    a, b = a[keep], b[keep]
    d = D.stage_distances(x, a, b)
    f = D.stage_qbound(x, a, b, d * np.float32(0.9))
    assert f.mean() > 0.95


def test_bound_rejects_unsupported_rows():
    with pytest.raises(D.BuildError):
        D.stage_qbound(np.zeros((10, 8), np.uint8), np.zeros(1, np.uint32), np.zeros(1, np.uint32),
                       np.zeros(1, np.float32))
    with pytest.raises(D.BuildError):  # 113 dims do not fit one code row
        D.stage_qbound(np.ones((10, 113), np.float32), np.zeros(1, np.uint32), np.zeros(1, np.uint32),
                       np.zeros(1, np.float32))


class _env:
    def __init__(self, **kv):
        self.kv = kv

    def __enter__(self):
        self.old = {k: os.environ.get(k) for k in self.kv}
        os.environ.update({k: str(v) for k, v in self.kv.items()})

    def __exit__(self, *exc):
        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def test_search_stage_on_adversarial_rows():
    x = adversarial(3000, 96, seed=21)
    R, L, C, steps = 32, 64, 48, 48
    s0 = O.init_graph(x, R, C)
    start, _, _ = O.medoid(x)
    from test_gpu_parity import assert_state_equal, to_dance
    want = O.search(x, s0, L, steps, 1.2, start)
    for env in ({}, {"DANCE_QBOUND": "0"}):
        with _env(**env):
            g = D.stage_search(x, to_dance(s0), L, steps, 1.2, start)
        assert_state_equal(g, want, ("work", "deg_work", "wd"))


@pytest.mark.parametrize("alpha", [1.0, 1.2, 2.0])
@pytest.mark.parametrize("C", [80, 150])
def test_prune_stage_on_adversarial_rows(alpha, C):
    """Candidate lists longer than one wave (C = 150) and both min-degree modes."""
    from test_gpu_parity import assert_state_equal, random_work_state, to_dance
    x = adversarial(2500, 96, seed=41)
    s0 = random_work_state(x, 32, C, seed=43)
    for md in (0, 32):
        want = O.prune(x, s0, md, alpha)
        for env in ({}, {"DANCE_QBOUND": "0"}):
            with _env(**env):
                g = D.stage_prune(x, to_dance(s0), md, alpha)
            assert_state_equal(g, want)


@pytest.mark.parametrize("profile", ["QUALITY", "FAST_SMALL"])
def test_build_identical_with_bound_off_first_and_every_iteration(profile):
    """QUALITY builds on fp32 rows, FAST_SMALL on the same input stored as fp16."""
    x = adversarial(4000, 96, seed=31, huge=profile == "QUALITY")
    ox = x if profile == "QUALITY" else x.astype(np.float16)
    og, od, om = O.vnew2_build(ox, 32, 64, 48, 32)
    seen = {}
    try:
        D.set_profile(profile)
        for name, env in (("off", {"DANCE_QBOUND": "0"}), ("first", {}),
                          ("all", {"DANCE_QBOUND_ITERS": "15", "DANCE_QBOUND_PRUNE_ITERS": "15"}),
                          ("prune_none", {"DANCE_QBOUND_PRUNE_ITERS": "0"}),
                          ("insert_all", {"DANCE_QBOUND_ITERS": "15", "DANCE_INSERT_BOUND_ITERS": "15"}),
                          ("insert_none", {"DANCE_INSERT_BOUND_ITERS": "0"})):
            with _env(**env):
                res = D.vamana_build(x, 32, 64, 48, 32)
            assert res.medoid == om, name
            assert np.array_equal(res.degree, od), name
            assert np.array_equal(res.graph, og), name
            kp = res.kernel_profile
            seen[name] = (kp["bound_checks"], kp["bound_skips"], kp["prune_bound_checks"], kp["prune_bound_skips"],
                          kp["insert_bound_checks"], kp["insert_bound_skips"], kp["insert_bound_checks_iter"][0],
                          kp["insert_bound_checks_iter"][3])
    finally:
        D.set_profile("QUALITY")
    assert seen["off"] == (0,) * 8
    # the insert bound: iteration 0 by default, every iteration on request, never without the search bound
    assert seen["first"][4] > 0 and seen["first"][5] > 0 and seen["first"][6] == seen["first"][4]
    assert seen["insert_all"][7] > 0 and seen["insert_all"][4] > seen["first"][4]
    assert seen["insert_none"][4] == 0
    assert seen["first"][0] > 0 and seen["first"][1] > 0 and seen["first"][3] > 0
    assert seen["all"][0] > seen["first"][0]
    assert seen["prune_none"][2:4] == (0, 0)


@pytest.mark.parametrize("profile", ["QUALITY", "FAST_SMALL"])
def test_build_with_non_finite_rows(profile):
    """Rows holding inf, -inf and NaN among the adversarial ones: their
    distances are inf or NaN, which no pool selects and no prune keeps, with
    the bound on and off; the graph is the oracle's."""
    x = adversarial(3000, 96, seed=51, huge=profile == "QUALITY")
    x[100] = np.inf
    x[101, 3] = np.nan
    x[102, 5] = -np.inf
    x[103:110] = np.nan
    x[110, :2] = [np.inf, -np.inf]
    ox = x if profile == "QUALITY" else x.astype(np.float16)
    og, od, om = O.vnew2_build(ox, 32, 64, 48, 32)
    try:
        D.set_profile(profile)
        for env in ({}, {"DANCE_QBOUND": "0"}, {"DANCE_QBOUND_ITERS": "15", "DANCE_QBOUND_PRUNE_ITERS": "15",
                                                 "DANCE_INSERT_BOUND_ITERS": "15"}):
            with _env(**env):
                res = D.vamana_build(x, 32, 64, 48, 32)
            assert res.medoid == om, env
            assert np.array_equal(res.degree, od), env
            assert np.array_equal(res.graph, og), env
    finally:
        D.set_profile("QUALITY")


def isotropic(n, dim, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, dim))
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    return x.astype(np.float32)


@pytest.mark.parametrize("n,R,L,C,steps", [(6000, 64, 100, 80, 64), (3000, 32, 64, 48, 32)])
def test_last_iteration_bound_follows_candidate_count(n, R, L, C, steps):
    """With DANCE_QBOUND_ITERS unset the build adds the bound to the last
    search iteration exactly when the iteration before it computed more than
    24 candidate distances (exact ones plus those the bound skipped) per
    expansion; R64 isotropic rows cross that line, R32 rows (at most 32
    candidates per expansion, most already seen) do not. The graph is the
    oracle's either way, and an explicit mask keeps the last iteration exact."""
    x = isotropic(n, 96, seed=n + R)
    og, od, om = O.vnew2_build(x, R, L, C, steps)
    prof = {}
    for name, env in (("auto", {}), ("first", {"DANCE_QBOUND_ITERS": "1"})):
        with _env(**env):
            res = D.vamana_build(x, R, L, C, steps)
        assert res.medoid == om and np.array_equal(res.degree, od) and np.array_equal(res.graph, og), name
        prof[name] = res.kernel_profile
    a, f = prof["auto"], prof["first"]
    last = int(a["iterations"]) - 1
    cand = a["search_dist_iter"][last - 1] + a["bound_skips_iter"][last - 1]
    fired = cand > 24 * a["expansions_iter"][last - 1]
    assert fired == (R == 64)
    assert (a["bound_checks_iter"][last] > 0) == fired
    assert f["bound_checks_iter"][last] == 0 and f["bound_checks_iter"][0] > 0
    assert all(a["bound_checks_iter"][i] == 0 for i in range(1, last))
