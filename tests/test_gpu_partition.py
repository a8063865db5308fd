"""GPU shard assignment (dance_partition_assign; DiskANN
shard_data_into_clusters_only_ids, called from build_merged_vamana_index,
integrations/dance-diskann-78256bba.patch:1212-1260) against the CPU oracle:
identical center lists (order included) for float and uint8 rows, widths up to
the 255 limit, k_base 1..8, duplicate centers, row counts that are not a
multiple of the 64-point workgroup and a run across the 4M-point upload chunk."""
import numpy as np
import pytest

from dance_amd import partition as P
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind,n,dim,K,k_base", [
    ("f32", 20000, 96, 37, 2), ("f32", 1000, 7, 3, 3), ("u8", 12345, 128, 40, 2), ("u8", 5000, 192, 11, 8),
    ("u8", 777, 255, 9, 1), ("f32", 65, 1, 8, 4),
])
def test_assign_matches_oracle(kind, n, dim, K, k_base):
    rng = np.random.default_rng(n + dim)
    if kind == "f32":
        x = rng.standard_normal((n, dim)).astype(np.float32)
        c = x[rng.choice(n, K, replace=False)] + 0.01 * rng.standard_normal((K, dim)).astype(np.float32)
    else:
        x = rng.integers(0, 256, (n, dim)).astype(np.uint8)
        c = x[rng.choice(n, K, replace=False)].astype(np.float32)
    c[-1] = c[0]  # duplicate center: the lower index wins ties
    got = P.assign(x, c, k_base)
    assert np.array_equal(got, O.partition_assign(x, c, k_base))


def test_assign_integer_ties_across_upload_chunks():
    # 4M + 100 points (one more upload than the 4M-point chunk), tiny integer
    # rows so that exact ties are everywhere
    rng = np.random.default_rng(5)
    n = (1 << 22) + 100
    x = rng.integers(0, 3, (n, 2)).astype(np.uint8)
    c = np.array([[0, 0], [1, 1], [2, 2], [1, 1], [0, 2]], np.float32)
    got = P.assign(x, c, 2)
    assert np.array_equal(got, O.partition_assign(x, c, 2))
