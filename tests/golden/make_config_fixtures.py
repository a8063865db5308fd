"""Writes tests/golden/config_fixtures.json: SHA-256 digests of the CPU
oracle's graphs on the BASELINE configurations' own generators, at sizes the
GPU tests rebuild on the device (tests/test_gpu_configs.py compares digests).

Each case records the digest of its input rows (so a failure can tell a
changed input from a changed graph) and of the oracle's output: graph rows
(N x R uint32, INVALID-padded), degrees and the entry point(s).

    python tests/golden/make_config_fixtures.py [case ...]

The oracle runs on all host cores; c2_1m takes a few minutes on 8 cores.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import dance_amd as D  # noqa: E402  (host-side generators only)
from dance_amd import INVALID  # noqa: E402
from dance_amd import filtered as F  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "config_fixtures.json")

# c5 parameters
C5 = dict(dim=192, centers=1024, sigma=0.3, vocab=20_000, R=64, L=100, FL=100, C=750, STEPS=64, alpha=1.2,
          parts=100, Rsmall=32, Lsmall=100, Rstitched=64, Cs=96)


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode() + str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def standard_case(cfg_name: str, n: int, iters: int = 4):
    """vnew2 build of the first n rows of a standard config's generator
    (iters: the reference's VAMANA_ITERS, DANCE_VAMANA_ITERS on the GPU)."""
    cfg = D.CONFIGS[cfg_name]
    base, _ = D.make_workload(cfg, n=n)
    g, d, m = O.vnew2_build(base, cfg["R"], cfg["L"], cfg["C"], cfg["STEPS"], iters=iters)
    return {"config": cfg_name, "n": n, "iters": iters, "input": digest(base),
            "graph": digest(g, d, np.array([m], np.uint32)),
            "medoid": int(m), "degree_sum": int(d.sum())}


def c5_rows(n: int) -> np.ndarray:
    return D.synth_u8(42, 0, n, C5["dim"], C5["centers"], C5["sigma"])


def c5_labels(n: int):
    return F.synth_labels(n, C5["vocab"], 1, 8, 1.0, seed=42)


def filtered_case(n: int):
    x = c5_rows(n)
    ls = c5_labels(n)
    starts = F.label_starts(x, ls)
    gs = F.global_start(x)
    rc, g, d, diag = O.filtered_build(x, ls.offsets, ls.labels, starts, ls.num_labels, C5["R"], C5["L"], C5["FL"],
                                      C5["C"], C5["STEPS"], C5["alpha"], INVALID, gs, 3)
    assert rc == 0
    return {"config": "c5-filtered", "n": n, "input": digest(x, ls.offsets, ls.labels, starts,
                                                              np.array([gs], np.uint32)),
            "graph": digest(g, d), "degree_sum": int(d.sum()), "diagnostics": [int(v) for v in diag]}


def stitched_partition(n: int) -> np.ndarray:
    """One of 100 labels per row, uniform (the c5 stitched partition)."""
    return np.random.default_rng(44).integers(0, C5["parts"], n).astype(np.uint32)


def stitched_case(n: int):
    """Per-label standard builds (Rsmall, Lsmall, C 96, steps 64) of the c5
    rows, remapped to global ids: row ids[i] holds ids[local neighbours]."""
    x = c5_rows(n)
    part = stitched_partition(n)
    graph = np.full((n, C5["Rstitched"]), INVALID, np.uint32)
    deg = np.zeros(n, np.uint32)
    medoids = np.full(C5["parts"], INVALID, np.uint32)
    for l in range(C5["parts"]):
        ids = np.nonzero(part == l)[0].astype(np.uint32)
        if ids.size == 0:
            continue
        g, d, m = O.vnew2_build(np.ascontiguousarray(x[ids]), C5["Rsmall"], C5["Lsmall"], C5["Cs"], C5["STEPS"])
        k = min(C5["Rsmall"], C5["Rstitched"])
        for i in range(ids.size):
            row = g[i, :d[i]]
            row = row[row < ids.size]
            graph[ids[i], :row.size] = ids[row]
            deg[ids[i]] = row.size
        medoids[l] = ids[m]
        del k
    return {"config": "c5-stitched", "n": n, "input": digest(x, part), "graph": digest(graph, deg, medoids),
            "degree_sum": int(deg.sum())}


CASES = {
    "c1_100k": lambda: standard_case("c1", 100_000),
    "c1_100k_iters5": lambda: standard_case("c1", 100_000, iters=5),
    "c2_1m": lambda: standard_case("c2", 1_000_000),
    "c3_200k": lambda: standard_case("c3", 200_000),
    "c4_200k": lambda: standard_case("c4", 200_000),
    "c5f_50k": lambda: filtered_case(50_000),
    "c5s_1m": lambda: stitched_case(1_000_000),
}


def main(names) -> None:
    old = {}
    if os.path.exists(OUT):
        with open(OUT) as f:
            old = json.load(f)
    for name in names or list(CASES):
        t0 = time.time()
        old[name] = CASES[name]()
        old[name]["oracle_seconds"] = round(time.time() - t0, 1)
        print(f"{name}: {old[name]}", flush=True)
        with open(OUT, "w") as f:
            json.dump(old, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main(sys.argv[1:])
