"""Builds dance_amd/libdance_hip.so and libdance_hip.a (gfx950) and the CLI
apps in-tree. The archive holds the same objects, for callers that link the
builders statically (as DANCE's CMake links its CUDA builder libraries).

The HIP sources are compiled with hipcc for gfx950 only. Flags that matter:
  -ffp-contract=off   the canonical distance uses explicit fmaf only
  -packed-fp32-ops    disabled (v_pk_*_f32 are not generated)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
APPS = os.path.join(HERE, "apps")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libdance_hip.so")
ARCHIVE = os.path.join(HERE, "libdance_hip.a")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-parameter", "-Wno-unused-function",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-pthread", "-Wall", "-Wextra", "-Wno-unused-parameter"]

HIP_SOURCES = ["vnew2_build.hip", "filtered_build.hip", "query_search.hip", "merge_shards.hip", "partition.hip"]
HOST_SOURCES = ["synth.cpp"]
APP_SOURCES = ["gpu_vamana_memory_index.cpp", "gpu_stitched_vamana_index.cpp", "build_memory_index.cpp",
               "build_sharded_index.cpp"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


def build(jobs: int | None = None) -> str:
    os.makedirs(OBJ, exist_ok=True)
    steps = []
    for src in HIP_SOURCES:
        obj = os.path.join(OBJ, src + ".o")
        steps.append(([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj], obj))
    for src in HOST_SOURCES:
        obj = os.path.join(OBJ, src + ".o")
        steps.append((["g++", *HOST_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj], obj))
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda s: _run(s[0]), steps))
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *[o for _, o in steps], "-o", tmp, "-pthread"])
    os.replace(tmp, LIB)
    tmp_a = ARCHIVE + ".tmp"
    if os.path.exists(tmp_a):
        os.remove(tmp_a)
    _run(["ar", "rcs", tmp_a, *[o for _, o in steps]])
    os.replace(tmp_a, ARCHIVE)
    for src in APP_SOURCES:
        path = os.path.join(APPS, src)
        if os.path.exists(path):
            exe = os.path.join(HERE, os.path.splitext(src)[0])
            _run(["g++", *HOST_FLAGS, "-fopenmp", f"-I{os.path.join(ROOT, 'include')}", path, "-o", exe,
                  f"-L{HERE}", "-ldance_hip", f"-Wl,-rpath,{HERE}", "-Wl,-rpath,$ORIGIN",
                  "-L/opt/rocm/lib", "-lamdhip64"])
    return LIB


if __name__ == "__main__":
    print(build())
