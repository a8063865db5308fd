"""Pins the CPU oracle of the shard assignment (oracle/partition_oracle.cpp;
DiskANN shard_data_into_clusters_only_ids, called from
build_merged_vamana_index, integrations/dance-diskann-78256bba.patch:1212-1260)
without sharing code with it:
  - integer-valued rows and centers: exact int64 squared distances and a
    stable sort by (distance, center index), ties included;
  - float rows: exact rational distances (fractions) wherever consecutive
    picks are not within a relative 1e-9 of each other;
  - a row of NaN gets no center."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O

INV = 0xFFFFFFFF


def exact_topk(x, c, k):
    d = ((x[:, None, :].astype(np.int64) - c[None, :, :].astype(np.int64)) ** 2).sum(-1)
    return np.argsort(d, axis=1, kind="stable")[:, :k].astype(np.uint32)


@pytest.mark.parametrize("seed,n,dim,K,k_base", [(1, 300, 8, 5, 2), (2, 200, 32, 17, 3), (3, 129, 3, 40, 8),
                                                 (4, 64, 1, 9, 1)])
def test_integer_rows_match_exact_order(seed, n, dim, K, k_base):
    rng = np.random.default_rng(seed)
    x = rng.integers(0, 6, (n, dim)).astype(np.uint8)  # small range: many exact ties
    c = rng.integers(0, 6, (K, dim)).astype(np.float32)
    c[K // 2] = c[0]  # a duplicate center: the lower index comes first
    got = O.partition_assign(x, c, k_base)
    assert np.array_equal(got, exact_topk(x, c, k_base))
    # the same rows as float32 give the same result
    assert np.array_equal(O.partition_assign(x.astype(np.float32), c, k_base), got)


def test_float_rows_match_exact_rational_order():
    rng = np.random.default_rng(7)
    n, dim, K, k_base = 40, 6, 12, 3
    x = rng.standard_normal((n, dim)).astype(np.float32)
    c = rng.standard_normal((K, dim)).astype(np.float32)
    got = O.partition_assign(x, c, k_base)
    checked = 0
    for i in range(n):
        d = [sum((Fraction(float(a)) - Fraction(float(b))) ** 2 for a, b in zip(x[i], c[k])) for k in range(K)]
        order = sorted(range(K), key=lambda k: (d[k], k))
        if any(abs(d[order[r + 1]] - d[order[r]]) <= Fraction(1, 10 ** 9) * d[order[r]] for r in range(k_base)):
            continue  # a near-tie: fp64 rounding may decide it either way
        assert got[i].tolist() == order[:k_base]
        checked += 1
    assert checked > n // 2


def test_nan_row_gets_no_center():
    x = np.ones((3, 4), np.float32)
    x[1] = np.nan
    c = np.zeros((5, 4), np.float32)
    got = O.partition_assign(x, c, 2)
    assert got[1].tolist() == [INV, INV] and got[0].tolist() == [0, 1]
