"""C-ABI checks that need no GPU: the library loads, exports every symbol the
headers declare with the reference's struct layout, rejects bad parameters
before touching the device, and the synthetic generators are deterministic."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import dance_amd as D

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = set()
    for h in ("gpu_vamana_builder.h", "gpu_vamana_filtered.h", "dance_hip.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b([a-z_0-9]+)\s*\(", text):
            n = m.group(1)
            if n.startswith(("gpu_vamana", "dance_")):
                names.add(n)
    return names


def test_library_exports_every_declared_symbol():
    lib = D.lib()
    declared = header_functions()
    assert declared == set(D.EXPORTS)
    out = subprocess.run(["nm", "-D", "--defined-only", D.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = declared - exported
    assert not missing, missing
    for n in declared:
        getattr(lib, n)


def test_static_archive_defines_every_declared_symbol(tmp_path):
    """libdance_hip.a (the same objects as the shared library) defines every
    declared entry point, and a C caller links against it statically."""
    archive = os.path.join(os.path.dirname(D.LIB_PATH), "libdance_hip.a")
    assert os.path.exists(archive), "build() writes the archive beside the shared library"
    out = subprocess.run(["nm", "--defined-only", archive], capture_output=True, text=True).stdout
    defined = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = header_functions() - defined
    assert not missing, missing
    src = tmp_path / "caller.c"
    src.write_text('#include "gpu_vamana_builder.h"\n#include "gpu_vamana_filtered.h"\n'
                   "int main(void) { GPUVamanaStats s; GPUFilteredVamanaStats f;\n"
                   "  gpu_vamana_vnew2_get_last_stats(&s); gpu_vamana_filtered_get_last_stats(&f);\n"
                   "  return (int)gpu_vamana_vnew2_get_last_medoid(); }\n")
    exe = tmp_path / "caller"
    r = subprocess.run(["g++", "-x", "c", str(src), "-x", "none", "-I", os.path.join(ROOT, "include"), archive,
                        "-L/opt/rocm/lib", "-lamdhip64", "-pthread", "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]


STATIC_CALLER = r"""
#include <stdio.h>
#include <stdlib.h>
#include "gpu_vamana_builder.h"
/* caller N dim R L C STEPS in.u8 out.graph out.degree */
int main(int argc, char** argv) {
  if (argc != 10) return 2;
  const uint32_t N = atoi(argv[1]), dim = atoi(argv[2]), R = atoi(argv[3]), L = atoi(argv[4]),
                 C = atoi(argv[5]), S = atoi(argv[6]);
  uint8_t* x = malloc((size_t)N * dim);
  uint32_t* g = malloc((size_t)N * R * 4);
  uint32_t* d = malloc((size_t)N * 4);
  FILE* f = fopen(argv[7], "rb");
  if (!f || fread(x, 1, (size_t)N * dim, f) != (size_t)N * dim) return 3;
  fclose(f);
  if (gpu_vamana_vnew2_build(x, N, dim, R, L, C, S, g, d) != 0) return 4;
  f = fopen(argv[8], "wb");
  fwrite(g, 4, (size_t)N * R, f);
  fclose(f);
  f = fopen(argv[9], "wb");
  fwrite(d, 4, N, f);
  fclose(f);
  printf("%u\n", gpu_vamana_vnew2_get_last_medoid());
  return 0;
}
"""


@pytest.mark.gpu
def test_static_archive_build_equals_oracle(tmp_path):
    """A C program linked against libdance_hip.a (no shared library) builds a
    graph on the GPU, identical to the oracle's."""
    from oracle import oracle as O
    archive = os.path.join(os.path.dirname(D.LIB_PATH), "libdance_hip.a")
    src = tmp_path / "caller.c"
    src.write_text(STATIC_CALLER)
    exe = tmp_path / "caller"
    r = subprocess.run(["g++", "-x", "c", str(src), "-x", "none", "-I", os.path.join(ROOT, "include"), archive,
                        "-L/opt/rocm/lib", "-lamdhip64", "-pthread", "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "libdance_hip" not in subprocess.run(["ldd", str(exe)], capture_output=True, text=True).stdout
    N, dim, R, L, Cc, S = 1500, 64, 32, 64, 48, 32
    x = np.random.default_rng(5).integers(0, 256, (N, dim), dtype=np.uint8)
    x.tofile(tmp_path / "x.u8")
    r = subprocess.run([str(exe), *map(str, (N, dim, R, L, Cc, S)), str(tmp_path / "x.u8"), str(tmp_path / "g.u32"),
                        str(tmp_path / "d.u32")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    g = np.fromfile(tmp_path / "g.u32", np.uint32).reshape(N, R)
    d = np.fromfile(tmp_path / "d.u32", np.uint32)
    og, od, om = O.vnew2_build(x, R, L, Cc, S)
    assert int(r.stdout.strip()) == om
    assert np.array_equal(d, od)
    assert np.array_equal(g, og)


def test_merge_cpp_symbol_exported():
    """include/gpu_merge.h declares diskann::merge_shards_gpu with std::string
    arguments (reference include/gpu_merge.h:8-12): the C++ symbol is exported."""
    out = subprocess.run(["nm", "-DC", "--defined-only", D.LIB_PATH], capture_output=True, text=True).stdout
    sym = [l for l in out.splitlines() if " T " in l and "diskann::merge_shards_gpu(" in l]
    assert len(sym) == 1, sym
    assert sym[0].count("std::__cxx11::basic_string") == 6 and "unsigned long, unsigned int" in sym[0]
    from dance_amd.merge import DanceMergeStats
    assert C.sizeof(DanceMergeStats) == 112 and DanceMergeStats.total_seconds.offset == 104


def test_merge_missing_inputs_before_device(tmp_path):
    """merge_shards_gpu validates id maps and headers before any device call."""
    from dance_amd import merge as M
    pre = (str(tmp_path / "s_"), ".index", str(tmp_path / "m_"), ".bin")
    assert M.merge_shards(*pre, 2, 8, str(tmp_path / "o"), str(tmp_path / "med")) == -2
    M.write_idmap(str(tmp_path / "m_0.bin"), [0, 1])
    M.write_idmap(str(tmp_path / "m_1.bin"), [1, 2])
    assert M.merge_shards(*pre, 2, 8, str(tmp_path / "o"), str(tmp_path / "med")) == -3
    M.write_shard(str(tmp_path / "s_0.index"), [[1], [0]], 5)
    M.write_shard(str(tmp_path / "s_1.index"), [[1], [0]], 0)
    assert M.merge_shards(*pre, 2, 8, str(tmp_path / "o"), str(tmp_path / "med")) == -4
    M.write_shard(str(tmp_path / "s_0.index"), [[1], [0]], 0, frozen=1)
    assert M.merge_shards(*pre, 2, 8, str(tmp_path / "o"), str(tmp_path / "med")) == -3
    M.write_shard(str(tmp_path / "s_0.index"), [[1], [0]], 0)
    raw = open(str(tmp_path / "s_1.index"), "rb").read()
    open(str(tmp_path / "s_1.index"), "wb").write(raw[:-4])
    assert M.merge_shards(*pre, 2, 8, str(tmp_path / "o"), str(tmp_path / "med")) == -6
    assert not os.path.exists(str(tmp_path / "o"))


def test_stats_struct_layout():
    assert C.sizeof(D.GPUVamanaStats) == 120
    assert D.GPUVamanaStats.distance_computations.offset == 56
    assert D.GPUVamanaStats.reverse_csr_seconds.offset == 104
    assert D.GPUVamanaStats.selective_active_nodes.offset == 112
    # GPUFilteredVamanaStats: 15 doubles, 29 u64, 4 doubles, u32 x5, double,
    # u32 x4, double, u32 x3 (reference include/gpu_vamana_filtered.h:11-77)
    F = D.GPUFilteredVamanaStats
    assert C.sizeof(F) == 456
    assert F.filtered_search_distance_count.offset == 120
    assert F.avg_common_label_out_degree.offset == 352
    assert F.out_degree_avg.offset == 408
    assert F.prune_output_degree_avg.offset == 432
    assert F.semantic_complete.offset == 448


def test_parameter_errors_return_minus_one():
    lib = D.lib()
    x = np.zeros((16, 8), np.float32)
    g = np.zeros((16, 8), np.uint32)
    deg = np.zeros(16, np.uint32)
    u32p = C.POINTER(C.c_uint32)
    gp, dp = g.ctypes.data_as(u32p), deg.ctypes.data_as(u32p)
    # null input, C < R, zero sizes: rejected before any device call
    assert lib.gpu_vamana_vnew2_build_float(None, 16, 8, 8, 16, 8, 8, gp, dp) == -1
    assert lib.gpu_vamana_vnew2_build_float(x.ctypes.data, 16, 8, 8, 16, 4, 8, gp, dp) == -1
    assert lib.gpu_vamana_vnew2_build_float(x.ctypes.data, 0, 8, 8, 16, 8, 8, gp, dp) == -1
    assert lib.gpu_vamana_vnew2_build(x.ctypes.data, 16, 8, 0, 16, 8, 8, gp, dp) == -1
    assert lib.gpu_vamana_build_float(x.ctypes.data, 16, 0, 8, 16, 8, 8, gp, dp) == -1
    assert lib.gpu_vamana_vnew2_build_float(x.ctypes.data, 16, 8, 8, 16, 8, 8, None, dp) == -1
    assert lib.dance_vamana_build_resident(None, 0, 16, 8, 8, 16, 8, 8, None, None) == -1
    assert lib.dance_set_profile(b"NOPE") == -1
    # build lists up to 1024 entries; more is rejected before any device call
    assert lib.gpu_vamana_vnew2_build_float(x.ctypes.data, 16, 8, 8, 1025, 8, 8, gp, dp) == -1
    # rows wider than 16 chunks of 16 bytes per lane are rejected before any device call
    wide = np.zeros((16, 513), np.float32)
    gw = np.zeros((16, 8), np.uint32)
    assert lib.gpu_vamana_vnew2_build_float(wide.ctypes.data, 16, 513, 8, 16, 8, 8,
                                            gw.ctypes.data_as(u32p), dp) == -1


@pytest.mark.parametrize("iters", ["0", "9", "four", "-1"])
def test_iteration_count_outside_range_is_an_error(iters, monkeypatch):
    """DANCE_VAMANA_ITERS (the reference's VAMANA_ITERS) takes 1..DANCE_MAX_ITERS;
    anything else fails validation with -1 before any device call."""
    monkeypatch.setenv("DANCE_VAMANA_ITERS", iters)
    lib = D.lib()
    x = np.zeros((16, 8), np.float32)
    g = np.zeros((16, 8), np.uint32)
    deg = np.zeros(16, np.uint32)
    u32p = C.POINTER(C.c_uint32)
    assert lib.gpu_vamana_vnew2_build_float(x.ctypes.data, 16, 8, 8, 16, 8, 8, g.ctypes.data_as(u32p),
                                            deg.ctypes.data_as(u32p)) == -1
    assert lib.gpu_vamana_build_float(x.ctypes.data, 16, 8, 8, 16, 8, 8, g.ctypes.data_as(u32p),
                                      deg.ctypes.data_as(u32p)) == -1
    assert D.MAX_ITERS == 8


def test_partition_assign_errors_before_device():
    from dance_amd import partition as P
    x = np.zeros((10, 8), np.float32)
    c = np.zeros((4, 8), np.float32)
    assert P.assign_rc(x, c, 0)[0] == -1            # k_base 0
    assert P.assign_rc(x, c, 5)[0] == -1            # k_base > centers
    assert P.assign_rc(x, np.zeros((20, 8), np.float32), 9)[0] == -1  # k_base > 8
    assert P.assign_rc(np.zeros((10, 256), np.float32), np.zeros((4, 256), np.float32), 2)[0] == -1  # dim > 255
    assert P.assign_rc(np.zeros((0, 8), np.float32), c, 2)[0] == 0  # no points: nothing to do
    with pytest.raises(TypeError):
        P.assign_rc(x.astype(np.float64), c, 1)


def test_filtered_parameter_errors():
    """Filtered ABI: -1 for null pointers, zero sizes, C < R and malformed
    label offsets; 1 when min(C, 128) < 2R (reference
    src/gpu_vamana_filtered.cu:6558-6568, 5839-5846). All are decided before
    any device call."""
    from dance_amd import filtered as F
    x = np.zeros((16, 8), np.uint8)
    xf = np.zeros((16, 8), np.float32)
    ls = F.LabelSet(np.arange(17, dtype=np.uint32), np.zeros(16, np.uint32), 1)
    st = np.zeros(1, np.uint32)
    assert F.build_rc(None, ls, st, 8, 16, 16, 64) == -1                 # null data
    assert F.build_rc(x, ls, st, 8, 16, 16, 4) == -1                     # C < R
    assert F.build_rc(x, ls, st, 0, 16, 16, 64) == -1                    # R = 0
    assert F.build_rc(x, ls, st, 8, 0, 16, 64) == -1                     # L = 0
    assert F.build_rc(x[:, :0].copy(), ls, st, 8, 16, 16, 64) == -1      # dim = 0
    assert F.build_rc(x, ls, st, 8, 16, 16, 64, total=15) == -1          # offsets[N] != total
    bad = F.LabelSet(np.r_[np.arange(9), np.arange(7, 15)].astype(np.uint32), np.zeros(16, np.uint32), 1)
    assert F.build_rc(x, bad, st, 8, 16, 16, 64, total=14) == -1         # offsets decrease
    # point 0 carries labels [3, 1] (not ascending), points 1..15 label 0
    unsorted = F.LabelSet(np.r_[0, np.arange(2, 18)].astype(np.uint32), np.r_[3, 1, np.zeros(15)].astype(np.uint32), 4)
    assert unsorted.offsets.shape[0] == 17 and unsorted.offsets[-1] == unsorted.labels.shape[0]
    assert F.build_rc(x, unsorted, np.zeros(4, np.uint32), 8, 16, 16, 64) == -1  # labels not ascending
    assert F.build_rc(x, ls, st, 40, 16, 16, 64) == 1                    # min(C,128) < 2R
    assert F.build_rc(xf, ls, st, 70, 16, 16, 750) == 1                  # 128 < 140
    assert F.build_rc(x, ls, st, 8, 16, 16, 64, rounds=4) == -1          # extension: rounds <= 3


def test_profiles():
    for p in ("FAST_SMALL", "PRO6000_100M", "FILTERED_PAPER", "QUALITY"):
        D.set_profile(p)
        assert D.get_profile() == p


def test_synth_deterministic_and_shaped():
    a = D.synth_f32(42, 0, 5000, 96, 256, 0.3, True)
    b = D.synth_f32(42, 0, 5000, 96, 256, 0.3, True)
    assert np.array_equal(a, b)
    assert np.allclose(np.linalg.norm(a, axis=1), 1.0, atol=1e-5)
    # rows do not depend on N (each row has its own stream)
    c = D.synth_f32(42, 0, 100, 96, 256, 0.3, True)
    assert np.array_equal(a[:100], c)
    # queries use another stream
    q = D.synth_f32(42, 1, 100, 96, 256, 0.3, True)
    assert not np.array_equal(q, c)
    u = D.synth_u8(42, 0, 3000, 128, 1024, 0.3)
    assert u.dtype == np.uint8 and u.shape == (3000, 128)
    assert 40 < u.mean() < 90
    g = D.synth_f32(42, 0, 20000, 16, 0, 1.0, False)
    assert abs(g.mean()) < 0.02 and abs(g.std() - 1.0) < 0.02


def test_mixture_is_clustered():
    x = D.synth_f32(42, 0, 4000, 96, 8, 0.3, True)
    # 8 well-separated components: nearest neighbours are far closer than random pairs
    d_rand = ((x[:200] - x[200:400]) ** 2).sum(1).mean()
    d_nn = min(((x[1:] - x[0]) ** 2).sum(1))
    assert d_nn < 0.5 * d_rand
