"""The v8 builder's oracle (gpu_vamana_uint8.cu:2437-3120) on the CPU.

The v8 oracle keeps the reference's own buffer scheme (two C-stride graphs, one
distance array, in-place reverse merge and prune, a swap per iteration), which
vnew2's oracle does not share. The pins:
  * it equals the vnew2 composition without the reverse heavy cap on u8, f32
    and f16 rows, under both alpha schedules: v8's kernels compute what vnew2's
    do (uint8.cu:1123-1540 vs vnew2.cu:1119-1439; :1795-1940 vs :1722-1814 with
    ENABLE_REVERSE_HEAVY_CAP=0; :2020-2298 vs :1893-2147);
  * it differs from vnew2 with the PRO6000_100M / FILTERED_PAPER cap (256/384)
    on data whose reverse lists exceed the threshold, so a v8 restatement that
    applied the cap fails here;
  * the parameter checks of uint8.cu:2443-2466 (null, zeros, C < R) and the
    STEPS > L clamp.
"""
import numpy as np
import pytest

from oracle import oracle as O


def data(kind, n, dim, seed=11):
    rng = np.random.default_rng(seed)
    if kind == "u8":
        return rng.integers(0, 256, (n, dim), dtype=np.uint8)
    x = rng.standard_normal((n, dim))
    return x.astype(np.float16 if kind == "f16" else np.float32)


@pytest.mark.parametrize("kind,n,dim,R,L,C,steps,alpha_from", [
    ("u8", 2000, 32, 32, 50, 48, 32, None),
    ("f32", 1500, 24, 24, 40, 40, 40, None),
    ("f16", 800, 20, 16, 30, 32, 30, None),
    ("u8", 1200, 16, 16, 80, 24, 70, 0),
    ("f32", 60, 8, 8, 16, 8, 16, 1),
])
def test_v8_equals_vnew2_without_heavy_cap(kind, n, dim, R, L, C, steps, alpha_from):
    x = data(kind, n, dim)
    g8, d8, m8 = O.v8_build(x, R=R, L=L, C_=C, STEPS=steps, alpha_from=alpha_from)
    g2, d2, m2 = O.vnew2_build(x, R=R, L=L, C_=C, STEPS=steps, alpha_from=alpha_from)
    assert m8 == m2
    assert np.array_equal(d8, d2)
    assert np.array_equal(g8, g2)
    assert (d8 <= R).all() and (d8 > 0).all()


def test_v8_has_no_heavy_cap():
    x = data("u8", 2000, 32)
    g8, d8, _ = O.v8_build(x, R=32, L=50, C_=48, STEPS=32)
    gc, dc, _ = O.vnew2_build(x, R=32, L=50, C_=48, STEPS=32, heavy_threshold=256, heavy_sample=384)
    assert not (np.array_equal(g8, gc) and np.array_equal(d8, dc))


def test_v8_parameter_checks():
    x = data("u8", 50, 8)
    for kw in (dict(R=16, C_=8), dict(R=0), dict(L=0), dict(STEPS=0), dict(C_=0)):
        args = dict(R=8, L=16, C_=16, STEPS=8)
        args.update(kw)
        with pytest.raises(ValueError):
            O.v8_build(x, **args)
    a = O.v8_build(x, R=8, L=16, C_=16, STEPS=40)
    b = O.v8_build(x, R=8, L=16, C_=16, STEPS=16)
    assert all(np.array_equal(p, q) for p, q in zip(a[:2], b[:2])) and a[2] == b[2]


def test_v8_single_point_and_pair():
    g, d, m = O.v8_build(data("f32", 1, 4), R=4, L=8, C_=4, STEPS=4)
    assert d[0] == 0 and m == 0 and (g == 0xFFFFFFFF).all()
    g, d, m = O.v8_build(data("f32", 2, 4), R=4, L=8, C_=4, STEPS=4)
    assert list(d) == [1, 1] and g[0, 0] == 1 and g[1, 0] == 0
