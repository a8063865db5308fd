"""gpu_vamana_memory_index app: argument and input errors (CPU), and a full
build written in DiskANN format (GPU)."""
import json
import os
import subprocess

import numpy as np
import pytest

import dance_amd as D
from dance_amd import formats
from oracle import oracle as O

APP = os.path.join(os.path.dirname(D.__file__), "gpu_vamana_memory_index")


def run_app(*args):
    return subprocess.run([APP, *args], capture_output=True, text=True, timeout=300)


@pytest.mark.parametrize("args,msg", [
    (["--bogus", "1"], "unknown argument"),
    (["--data_path"], "missing value"),
    (["--data_path", "x", "--index_prefix", "p", "--data_type", "int8"], "--data_type must be"),
    (["--data_path", "x", "--index_prefix", "p", "--R", "0"], "must be in [1, UINT32_MAX]"),
    (["--data_path", "x", "--index_prefix", "p", "--R", "12a"], "must be an unsigned integer"),
    (["--data_path", "x"], "requires --index_prefix"),
    (["--data_path", "x", "--index_prefix", "p", "--builder", "v8"], "requires --builder vnew2"),
    (["--data_path", "/nonexistent/x.bin", "--index_prefix", "p"], "failed to open"),
])
def test_argument_errors(args, msg):
    r = run_app(*args)
    assert r.returncode == 2
    assert msg in r.stderr and "Usage:" in r.stderr


def test_input_file_errors(tmp_path):
    x = np.zeros((10, 4), np.float32)
    p = str(tmp_path / "x.bin")
    formats.write_bin(p, x)
    with open(p, "ab") as f:
        f.write(b"\0")  # one byte too many
    r = run_app("--data_path", p, "--data_type", "float", "--index_prefix", str(tmp_path / "i"))
    assert r.returncode == 2 and "does not match exact file size" in r.stderr
    formats.write_bin(p, x)
    r = run_app("--data_path", p, "--data_type", "float", "--index_prefix", str(tmp_path / "i"),
                "--offset", "8", "--npts", "5")
    assert r.returncode == 2 and "exceeds base file point count" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["float", "uint8"])
def test_build_writes_diskann_index(tmp_path, kind):
    rng = np.random.default_rng(3)
    if kind == "float":
        x = rng.standard_normal((3000, 96)).astype(np.float32)
    else:
        x = rng.integers(0, 256, (3000, 128), dtype=np.uint8)
    p = str(tmp_path / "x.bin")
    formats.write_bin(p, x)
    prefix = str(tmp_path / "idx")
    args = ["--data_path", p, "--data_type", kind, "--index_prefix", prefix, "--R", "32", "--L", "64",
            "--C", "48", "--STEPS", "32", "--offset", "500", "--npts", "2000"]
    r = run_app(*args)
    assert r.returncode == 0, r.stderr
    rep = json.loads(r.stdout)
    assert rep["graph_valid"] and rep["memory_index_serialized"] and rep["npts"] == 2000
    assert rep["invalid_neighbor_count"] == 0 and rep["self_loop_count"] == 0
    adj, max_deg, start, frozen = formats.read_graph(prefix)
    og, od, om = O.vnew2_build(np.ascontiguousarray(x[500:2500]), 32, 64, 48, 32)
    assert start == om == rep["medoid"] and frozen == 0
    assert max_deg == int(od.max())
    for v in range(2000):
        assert np.array_equal(adj[v], og[v, :od[v]])
    back = formats.read_bin(prefix + ".data", np.float32 if kind == "float" else np.uint8)
    assert np.array_equal(back, x[500:2500])
    # refuses to overwrite an existing index
    r2 = run_app(*args)
    assert r2.returncode == 2 and "refusing to overwrite" in r2.stderr
