"""build_sharded_index: the GPU shard path of DiskANN's
build_merged_vamana_index (integrations/dance-diskann-78256bba.patch:1209-1560).

CPU: option errors, decided before any device call.
GPU: given the centroids the app wrote, its shard id lists, shard graphs,
merged graph and medoid file equal an oracle pipeline built from the pinned
parts (oracle assignment, the oracle of the shard builder per shard: v8 by
default, vnew2 under DISKANN_GPU_VAMANA_VERSION=vnew2, at shard_R = 2R/3,
C = max(2 shard_R, shard_R + 32), STEPS = min(L, 20), the reference's shard
save format, oracle merge), byte for byte. The k-means that produces the
centroids restates DiskANN's upstream partitioner (absent): parity unpinned
there; the test checks its invariants (K finite rows, every point in k_base
distinct shards)."""
import os
import struct
import subprocess

import numpy as np
import pytest

import dance_amd as D
from dance_amd import formats
from oracle import oracle as O

APP = os.path.join(os.path.dirname(D.__file__), "build_sharded_index")


def run_app(*args, env=None):
    return subprocess.run([APP, *args], capture_output=True, text=True, timeout=900, env=env)


def make_data(tmp_path, kind, n, dim, seed):
    rng = np.random.default_rng(seed)
    if kind == "uint8":
        centers = rng.integers(40, 216, (12, dim))
        x = np.clip(centers[rng.integers(0, 12, n)] + rng.normal(0, 12, (n, dim)), 0, 255).astype(np.uint8)
    else:
        centers = rng.standard_normal((12, dim))
        x = (centers[rng.integers(0, 12, n)] + 0.3 * rng.standard_normal((n, dim))).astype(np.float32)
    path = str(tmp_path / "base.bin")
    formats.write_bin(path, x)
    return x, path


@pytest.mark.parametrize("extra,msg", [
    ([], "give --num_shards or a positive --budget_gb"),
    (["--num_shards", "4", "--k_base", "9"], "--k_base must be 1..8"),
    (["--num_shards", "1", "--k_base", "2"], "at least --k_base"),
    (["--num_shards", "4", "--data_type", "int8"], "uint8 or float"),
    (["--num_shards", "4", "--sampling_rate", "2"], "[0, 1]"),
    (["--num_shards", "4", "--bogus", "1"], "unknown argument"),
])
def test_option_errors(tmp_path, extra, msg):
    _, path = make_data(tmp_path, "uint8", 50, 8, 1)
    r = run_app("--data_type", "uint8", "--data_path", path, "--index_path_prefix", str(tmp_path / "idx"), *extra)
    assert r.returncode == 255 and msg in r.stderr, r.stderr


HEAVY = {"QUALITY": (0, 0), "FAST_SMALL": (0, 0), "PRO6000_100M": (256, 384), "FILTERED_PAPER": (256, 384)}


def shard_build(rows, builder, profile, **kw):
    """The oracle of one shard build: v8 (no heavy cap) or vnew2 with the
    profile's cap; float rows are stored as binary16 under the fp16 profiles."""
    if rows.dtype == np.float32 and profile != "QUALITY":
        rows = rows.astype(np.float16)
    if builder == "v8":
        return O.v8_build(rows, **kw)
    t, smp = HEAVY[profile]
    return O.vnew2_build(rows, heavy_threshold=t, heavy_sample=smp, **kw)


def oracle_pipeline(tmp_path, x, centroids, R, L, k_base, builder="v8", profile="QUALITY"):
    shard_R = 2 * R // 3
    C_ = max(2 * shard_R, shard_R + 32, shard_R)
    steps = min(L, 20)
    a = O.partition_assign(x, centroids, k_base)
    K = centroids.shape[0]
    pre = str(tmp_path / "oracle_sub-")
    ids_all = []
    for k in range(K):
        ids = np.nonzero((a == k).any(1))[0].astype(np.uint32)
        ids_all.append(ids)
        formats.write_bin(f"{pre}{k}_ids_uint32.bin", ids.reshape(-1, 1))
        body = bytearray()
        med = 0
        if ids.size:
            g, d, med = shard_build(x[ids], builder, profile, R=shard_R, L=L, C_=C_, STEPS=steps)
            med = med if med < ids.size else 0
            for i in range(ids.size):
                k_i = min(int(d[i]), shard_R)
                body += struct.pack("<I", k_i) + g[i, :k_i].astype("<u4").tobytes()
        with open(f"{pre}{k}_mem.index", "wb") as f:
            f.write(struct.pack("<QIIQ", 24 + len(body), shard_R, med, 0) + bytes(body))
    out, meds = str(tmp_path / "oracle.index"), str(tmp_path / "oracle_medoids.bin")
    rc, _ = O.merge_shards(pre, "_mem.index", pre, "_ids_uint32.bin", K, R, out, meds)
    assert rc == 0
    return ids_all, pre, out, meds


@pytest.mark.gpu
@pytest.mark.parametrize("kind,n,dim,R,L,shards,k_base", [("uint8", 6000, 32, 32, 50, 4, 2),
                                                          ("float", 5000, 24, 48, 60, 5, 2),
                                                          ("uint8", 3000, 16, 24, 40, 3, 1)])
def test_sharded_build_matches_oracle_pipeline(tmp_path, kind, n, dim, R, L, shards, k_base):
    x, path = make_data(tmp_path, kind, n, dim, n)
    prefix = str(tmp_path / "idx")
    r = run_app("--data_type", kind, "--data_path", path, "--index_path_prefix", prefix, "-R", str(R), "-L", str(L),
                "--num_shards", str(shards), "--k_base", str(k_base), "--sampling_rate", "0.5", "--seed", "7")
    assert r.returncode == 0, r.stdout + r.stderr
    cen = formats.read_bin(prefix + "_centroids.bin", np.float32)
    assert cen.shape == (shards, dim) and np.isfinite(cen).all()
    ids_all, pre, out, meds = oracle_pipeline(tmp_path, x, cen, R, L, k_base)
    counts = np.zeros(n, np.int64)
    for k, ids in enumerate(ids_all):
        got = formats.read_bin(f"{prefix}_tempFiles_subshard-{k}_ids_uint32.bin", np.uint32).ravel()
        assert np.array_equal(got, ids)
        counts[ids] += 1
        with open(f"{prefix}_tempFiles_subshard-{k}_mem.index", "rb") as f, open(f"{pre}{k}_mem.index", "rb") as g:
            assert f.read() == g.read(), f"shard {k} graph differs from the oracle's"
    assert (counts == k_base).all()
    with open(prefix, "rb") as f, open(out, "rb") as g:
        assert f.read() == g.read(), "merged graph differs from the oracle's"
    with open(prefix + "_medoids.bin", "rb") as f, open(meds, "rb") as g:
        assert f.read() == g.read()


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["uint8", "float"])
def test_sharded_builder_choice_under_heavy_cap_profile(tmp_path, kind):
    """Under PRO6000_100M the default shard builder is v8 (no heavy cap) and
    DISKANN_GPU_VAMANA_VERSION=vnew2 selects vnew2 (cap 256/384), as the
    patch's use_gpu_vamana_vnew2 (patch:2576-2584); each run equals the oracle
    pipeline of its builder, and the shard graphs of the two differ."""
    # Uniform rows: their k-NN graphs have hubs whose reverse lists pass 384.
    n, dim, R, L, shards, k_base = 6000, 32, 48, 60, 2, 1
    rng = np.random.default_rng(5)
    if kind == "uint8":
        x = rng.integers(0, 256, (n, dim), dtype=np.uint8)
    else:
        x = rng.standard_normal((n, dim)).astype(np.float32)
    path = str(tmp_path / "base.bin")
    formats.write_bin(path, x)
    outs = {}
    for builder in ("v8", "vnew2"):
        env = dict(os.environ, DANCE_PROFILE="PRO6000_100M")
        if builder == "vnew2":
            env["DISKANN_GPU_VAMANA_VERSION"] = "vnew2"
        prefix = str(tmp_path / f"idx_{builder}")
        print(f"sharded {kind} builder={builder}", flush=True)
        r = run_app("--data_type", kind, "--data_path", path, "--index_path_prefix", prefix, "-R", str(R), "-L",
                    str(L), "--num_shards", str(shards), "--k_base", str(k_base), "--sampling_rate", "0.5",
                    "--seed", "7", env=env)
        assert r.returncode == 0, r.stdout + r.stderr
        assert f"builder={builder}" in r.stdout
        cen = formats.read_bin(prefix + "_centroids.bin", np.float32)
        sub = tmp_path / f"oracle_{builder}"
        sub.mkdir()
        _, pre, out, meds = oracle_pipeline(sub, x, cen, R, L, k_base, builder, "PRO6000_100M")
        for k in range(shards):
            with open(f"{prefix}_tempFiles_subshard-{k}_mem.index", "rb") as f, open(f"{pre}{k}_mem.index", "rb") as g:
                assert f.read() == g.read(), f"{builder} shard {k} differs from its oracle"
        with open(prefix, "rb") as f, open(out, "rb") as g:
            outs[builder] = f.read()
            assert outs[builder] == g.read(), f"{builder} merged graph differs from its oracle"
    assert outs["v8"] != outs["vnew2"]


@pytest.mark.gpu
def test_sharded_budget_picks_the_number_of_shards(tmp_path):
    # a budget below one shard's estimate keeps adding two parts
    x, path = make_data(tmp_path, "uint8", 4000, 16, 3)
    prefix = str(tmp_path / "idx")
    r = run_app("--data_type", "uint8", "--data_path", path, "--index_path_prefix", prefix, "-R", "24", "-L", "40",
                "--budget_gb", "0.0006", "--sampling_rate", "0.5")
    assert r.returncode == 0, r.stdout + r.stderr
    cen = formats.read_bin(prefix + "_centroids.bin", np.float32)
    assert cen.shape[0] >= 5 and cen.shape[0] % 2 == 1
    assert "parts=3" in r.stdout
