"""GPU parity of the v8 builder's symbols, gpu_vamana_build[_float]
(gpu_vamana_uint8.cu:2437-3120), against the v8 oracle, bit for bit, under
every profile, including the profiles whose vnew2 build caps heavy reverse
lists (v8 never does)."""
import ctypes as C

import numpy as np
import pytest

import dance_amd as D
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def data(kind, n, dim, seed=11):
    rng = np.random.default_rng(seed)
    if kind == "u8":
        return rng.integers(0, 256, (n, dim), dtype=np.uint8)
    x = rng.standard_normal((n, dim)).astype(np.float32)
    return x / np.linalg.norm(x, axis=1, keepdims=True).astype(np.float32)


def with_profile(name, fn):
    D.set_profile(name)
    try:
        return fn()
    finally:
        D.set_profile("QUALITY")


@pytest.mark.parametrize("profile", ["QUALITY", "FAST_SMALL", "PRO6000_100M", "FILTERED_PAPER"])
@pytest.mark.parametrize("kind,n,dim,R,L,C,steps", [("u8", 2000, 32, 32, 50, 48, 32),
                                                    ("f32", 1500, 24, 24, 40, 40, 40),
                                                    ("f32", 700, 96, 64, 100, 80, 64)])
def test_v8_build_equals_v8_oracle(profile, kind, n, dim, R, L, C, steps):
    x = data(kind, n, dim)
    print(f"v8 build profile={profile} kind={kind} n={n} dim={dim} R={R} L={L} C={C}", flush=True)
    res = with_profile(profile, lambda: D.vamana_build(x, R, L, C, steps, entry="v8"))
    fp16 = profile != "QUALITY" and kind == "f32"
    og, od, om = O.v8_build(x.astype(np.float16) if fp16 else x, R=R, L=L, C_=C, STEPS=steps)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)
    assert res.stats["gpu_build_seconds"] > 0


def test_v8_differs_from_capped_vnew2():
    """Under PRO6000_100M the vnew2 entry caps reverse lists above 256 at 384
    samples and equals the capped vnew2 oracle; the v8 entry on the same input
    equals the uncapped v8 oracle, and the two graphs differ."""
    x = data("u8", 2000, 32)
    kw = dict(R=32, L=50, C_=48, STEPS=32)
    v2 = with_profile("PRO6000_100M", lambda: D.vamana_build(x, 32, 50, 48, 32, entry="vnew2"))
    v8 = with_profile("PRO6000_100M", lambda: D.vamana_build(x, 32, 50, 48, 32, entry="v8"))
    cg, cd, _ = O.vnew2_build(x, heavy_threshold=256, heavy_sample=384, **kw)
    g8, d8, _ = O.v8_build(x, **kw)
    assert np.array_equal(v2.graph, cg) and np.array_equal(v2.degree, cd)
    assert np.array_equal(v8.graph, g8) and np.array_equal(v8.degree, d8)
    assert not np.array_equal(v2.graph, v8.graph)


def test_v8_and_vnew2_getters_are_separate():
    """Each builder keeps its own last medoid and stats (the reference's two
    files hold file-static state each, uint8.cu:2416-2435)."""
    a = data("f32", 900, 16, seed=3)
    b = data("u8", 1100, 24, seed=4)
    ra = D.vamana_build(a, 16, 32, 24, 32, entry="vnew2")
    rb = D.vamana_build(b, 16, 32, 24, 32, entry="v8")
    _, _, ma = O.vnew2_build(a, R=16, L=32, C_=24, STEPS=32)
    _, _, mb = O.v8_build(b, R=16, L=32, C_=24, STEPS=32)
    assert ra.medoid == ma and rb.medoid == mb
    assert D.last_medoid("vnew2") == ma and D.last_medoid("v8") == mb
    assert D.last_stats("vnew2")["gpu_build_seconds"] == ra.stats["gpu_build_seconds"]
    assert D.last_stats("v8")["gpu_build_seconds"] == rb.stats["gpu_build_seconds"]


def test_v8_rejects_bad_parameters():
    x = data("u8", 64, 8)
    g = np.empty((64, 16), np.uint32)
    d = np.empty(64, np.uint32)
    lib = D.lib()
    gp, dp = (a.ctypes.data_as(C.POINTER(C.c_uint32)) for a in (g, d))
    assert lib.gpu_vamana_build(x.ctypes.data, 64, 8, 16, 32, 8, 16, gp, dp) == -1  # C < R
    assert lib.gpu_vamana_build(x.ctypes.data, 0, 8, 16, 32, 16, 16, gp, dp) == -1
    assert lib.gpu_vamana_build(None, 64, 8, 16, 32, 16, 16, gp, dp) == -1


@pytest.mark.parametrize("n", [1, 2, 17, 130])
def test_v8_tiny_inputs(n):
    """Tiny builds: one point (no neighbours), two points, rows shorter than R."""
    x = data("f32", n, 8, seed=n)
    res = D.vamana_build(x, 8, 16, 16, 8, entry="v8")
    og, od, om = O.v8_build(x, R=8, L=16, C_=16, STEPS=8)
    assert res.medoid == om
    assert np.array_equal(res.degree, od)
    assert np.array_equal(res.graph, og)
