"""GPU shard-graph merge (diskann::merge_shards_gpu, reference
src/gpu_merge.cu:351-790) against the CPU oracle: merged graph and medoid
files byte-identical, statistics equal, across degree caps, buckets, hub
sources whose edge lists exceed one wave's LDS sort, seeds and error codes."""
import os

import pytest

from dance_amd import merge as M
from oracle import oracle as O
from tests.merge_cases import make_shards, read_merged
from tests.test_merge_oracle import ERRORS, corrupt

pytestmark = pytest.mark.gpu


def both(tmp_path, pre, nshards, K, seed=O.MERGE_DEFAULT_SEED):
    go, gm = str(tmp_path / "gpu.index"), str(tmp_path / "gpu_medoids.bin")
    oo, om = str(tmp_path / "cpu.index"), str(tmp_path / "cpu_medoids.bin")
    rc_g = M.merge_shards(*pre, nshards, K, go, gm)
    stats = M.last_stats()
    rc_o, cnt = O.merge_shards(*pre, nshards, K, oo, om, seed)
    return rc_g, rc_o, stats, cnt, (go, gm, oo, om)


def assert_same(files):
    go, gm, oo, om = files
    assert open(go, "rb").read() == open(oo, "rb").read(), "merged graph differs from the oracle"
    assert open(gm, "rb").read() == open(om, "rb").read(), "medoid file differs from the oracle"


@pytest.mark.parametrize("seed,nnodes,nshards,width,K,gaps", [
    (1, 60, 1, 8, 64, False),
    (2, 200, 3, 24, 16, False),
    (3, 3000, 4, 40, 32, True),
    (4, 50, 6, 49, 7, False),
    (5, 120, 2, 10, 0, True),
    (6, 20000, 3, 64, 64, False),
    (7, 5000, 8, 32, 200, False),
])
def test_merge_matches_oracle(tmp_path, seed, nnodes, nshards, width, K, gaps):
    pre, _ = make_shards(tmp_path, seed, nnodes, nshards, width, gaps=gaps)
    rc_g, rc_o, st, cnt, files = both(tmp_path, pre, nshards, K)
    assert rc_g == 0 and rc_o == 0
    assert_same(files)
    assert st["self_loops"] == cnt["self_loops"]
    assert st["unique_edges"] == cnt["unique_edges"]
    assert st["output_edges"] == cnt["output_edges"]
    assert st["buckets"] == 1 and st["long_segments"] == 0


@pytest.mark.parametrize("buckets", ["2", "7", "1000"])
def test_merge_buckets_do_not_change_output(tmp_path, monkeypatch, buckets):
    pre, _ = make_shards(tmp_path, 21, 4000, 3, 32)
    monkeypatch.setenv("DISKANN_GPU_MERGE_BUCKETS", buckets)
    rc_g, rc_o, st, cnt, files = both(tmp_path, pre, 3, 24)
    assert rc_g == 0 and rc_o == 0
    assert st["buckets"] == int(buckets)
    assert_same(files)
    assert st["unique_edges"] == cnt["unique_edges"] and st["self_loops"] == cnt["self_loops"]


@pytest.mark.parametrize("K,hub_degree", [(64, 400), (3000, 700), (1, 300)])
def test_merge_long_segments(tmp_path, K, hub_degree):
    # the hub is in all 12 shards with up to hub_degree neighbours each: its
    # edge list (thousands) exceeds the 1024-key LDS sort and takes the radix path
    pre, _ = make_shards(tmp_path, 31, 3000, 12, 16, hub=17, hub_degree=hub_degree)
    rc_g, rc_o, st, cnt, files = both(tmp_path, pre, 12, K)
    assert rc_g == 0 and rc_o == 0
    assert st["long_segments"] >= 1
    assert_same(files)
    assert st["unique_edges"] == cnt["unique_edges"]


def test_merge_long_segments_across_buckets(tmp_path, monkeypatch):
    pre, _ = make_shards(tmp_path, 32, 2000, 10, 12, hub=1500, hub_degree=600)
    monkeypatch.setenv("DISKANN_GPU_MERGE_BUCKETS", "3")
    rc_g, rc_o, st, cnt, files = both(tmp_path, pre, 10, 48)
    assert rc_g == 0 and rc_o == 0 and st["long_segments"] >= 1
    assert_same(files)


def test_merge_seed_override(tmp_path, monkeypatch):
    pre, _ = make_shards(tmp_path, 41, 1000, 3, 30)
    monkeypatch.setenv("DISKANN_GPU_MERGE_HASH_SEED", "777")
    rc_g, rc_o, _, _, files = both(tmp_path, pre, 3, 5, seed=777)
    assert rc_g == 0 and rc_o == 0
    assert_same(files)


def test_merge_no_shards(tmp_path):
    pre = (str(tmp_path / "s"), ".i", str(tmp_path / "m"), ".b")
    rc_g, rc_o, st, _, files = both(tmp_path, pre, 0, 8)
    assert rc_g == 0 and rc_o == 0
    assert_same(files)
    assert st["nnodes"] == 0


@pytest.mark.parametrize("what,code", ERRORS)
def test_merge_error_codes(tmp_path, what, code):
    pre = corrupt(tmp_path, what)
    out = str(tmp_path / "gpu.index")
    assert M.merge_shards(*pre, 2, 8, out, str(tmp_path / "gpu_medoids.bin")) == code
    if code in (-2, -3, -4, -6, -7):
        assert not os.path.exists(out), "no output is written before the inputs are validated"


def test_merge_unwritable_outputs(tmp_path):
    pre, _ = make_shards(tmp_path, 51, 100, 2, 8)
    bad = str(tmp_path / "missing_dir" / "x")
    assert M.merge_shards(*pre, 2, 8, str(tmp_path / "o.index"), bad) == -10
    assert M.merge_shards(*pre, 2, 8, bad, str(tmp_path / "m.bin")) == -11


def test_merge_scale(tmp_path):
    # 200k global nodes in 4 shards of ~half the nodes each (the overlap of a
    # k-means sharded build), width 64: device passes and file I/O at scale.
    pre, _ = make_shards(tmp_path, 61, 200_000, 4, 64, cover=0.5, self_loop_p=0.0)
    rc_g, rc_o, st, cnt, files = both(tmp_path, pre, 4, 64)
    assert rc_g == 0 and rc_o == 0
    assert_same(files)
    print(f"[merge] 200k nodes: {st['input_edges']} input edges, device {st['device_ms']:.2f} ms, "
          f"read {st['read_seconds']:.3f} s, write {st['write_seconds']:.3f} s, total {st['total_seconds']:.3f} s")
    hdr, _ = read_merged(files[0])
    assert hdr["size"] == hdr["file_size"]
