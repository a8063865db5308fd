"""Pins the CPU oracle of the shard-graph merge (oracle/merge_oracle.cpp,
reference src/gpu_merge.cu:351-790) without sharing code with it:
  - mix64 against its closed-form inverse (modular inverses of the two
    multipliers, xor-shift 33 undone in one step);
  - the merged graph against tests/merge_cases.expected_merge (Python sets and
    sorted()) on random shard sets, with self loops, duplicates across shards,
    ids no shard carries and degree caps below and above the distinct count;
  - headers, the medoid file, and the reference's error codes."""
import os
import struct

import numpy as np
import pytest

from oracle import oracle as O
from tests.merge_cases import expected_merge, make_shards, read_medoids, read_merged

M64 = (1 << 64) - 1
C1, C2 = 0xFF51AFD7ED558CCD, 0xC4CEB9FE1A85EC53


def inverse_mix64(y: int) -> int:
    def unshift(v):  # v ^ (v >> 33) is its own inverse for shifts >= 32
        return v ^ (v >> 33)

    y = unshift(y)
    y = (y * pow(C2, -1, 1 << 64)) & M64
    y = unshift(y)
    y = (y * pow(C1, -1, 1 << 64)) & M64
    return unshift(y)


def test_mix64_is_the_inverted_bijection():
    rng = np.random.default_rng(5)
    xs = [0, 1, M64, 1 << 63, 0x9E3779B97F4A7C15] + [int(v) for v in rng.integers(0, 1 << 63, 200, dtype=np.int64)]
    for x in xs:
        assert inverse_mix64(O.mix64(x)) == x
    assert O.mix64(0) == 0


def test_edge_hash_folds_mix64():
    for src, dst, seed in [(0, 0, 0), (1, 2, O.MERGE_DEFAULT_SEED), (0xFFFFFFFE, 7, 12345), (99, 0xFFFFFFF0, 1)]:
        m = O.mix64(((src << 32) ^ dst ^ seed) & M64)
        assert O.edge_hash(src, dst, seed) == (m ^ (m >> 32)) & 0xFFFFFFFF


def run_oracle(tmp, pre, nshards, K, seed=O.MERGE_DEFAULT_SEED):
    out, med = os.path.join(str(tmp), "merged.index"), os.path.join(str(tmp), "medoids.bin")
    rc, cnt = O.merge_shards(*pre, nshards, K, out, med, seed)
    return rc, cnt, out, med


@pytest.mark.parametrize("seed,nnodes,nshards,width,K,gaps", [
    (1, 60, 1, 8, 64, False),
    (2, 200, 3, 24, 16, False),
    (3, 300, 4, 40, 32, True),
    (4, 50, 6, 49, 7, False),
    (5, 120, 2, 10, 0, True),
])
def test_oracle_merge_matches_definition(tmp_path, seed, nnodes, nshards, width, K, gaps):
    pre, shards = make_shards(tmp_path, seed, nnodes, nshards, width, gaps=gaps)
    rc, cnt, out, med = run_oracle(tmp_path, pre, nshards, K)
    assert rc == 0
    rows, medoids = expected_merge(shards, K, O.edge_hash)
    hdr, got = read_merged(out)
    assert got == rows
    assert hdr["size"] == hdr["file_size"] and hdr["width"] == K and hdr["frozen"] == 0
    assert hdr["medoid"] == medoids[-1]
    n, one, meds = read_medoids(med)
    assert (n, one, meds) == (nshards, 1, medoids)
    assert cnt["output_edges"] == sum(len(r) for r in rows)
    uniq = expected_merge(shards, 1 << 30, O.edge_hash)[0]
    assert cnt["unique_edges"] == sum(len(r) for r in uniq)
    loops = sum(int(np.sum(np.asarray(idmap)[np.asarray(nb, dtype=np.int64)] == idmap[r]))
                for idmap, adj, _ in shards for r, nb in enumerate(adj) if len(nb))
    assert cnt["self_loops"] == loops


def test_oracle_seed_changes_ranking(tmp_path):
    pre, shards = make_shards(tmp_path, 9, 100, 3, 30)
    rc, _, out, _ = run_oracle(tmp_path, pre, 3, 5, seed=777)
    assert rc == 0
    rows, _ = expected_merge(shards, 5, lambda s, d: O.edge_hash(s, d, 777))
    assert read_merged(out)[1] == rows


def test_oracle_no_shards(tmp_path):
    rc, cnt, out, med = run_oracle(tmp_path, (str(tmp_path / "s"), ".i", str(tmp_path / "m"), ".b"), 0, 8)
    assert rc == 0
    hdr, rows = read_merged(out)
    assert rows == [] and hdr["size"] == 24 and hdr["medoid"] == 0
    assert read_medoids(med) == (0, 1, [])


def corrupt(tmp_path, what):
    pre, shards = make_shards(tmp_path, 11, 80, 2, 12)
    vp, vs, ip, is_ = pre
    g1, m1 = f"{vp}1{vs}", f"{ip}1{is_}"
    if what == "missing_idmap":
        os.remove(m1)
    elif what == "idmap_dim":
        raw = bytearray(open(m1, "rb").read())
        raw[4:8] = struct.pack("<I", 2)
        open(m1, "wb").write(raw)
    elif what == "idmap_size":
        open(m1, "ab").write(b"\0\0\0\0")
    elif what == "missing_graph":
        os.remove(g1)
    elif what == "frozen":
        raw = bytearray(open(g1, "rb").read())
        raw[16:24] = struct.pack("<Q", 1)
        open(g1, "wb").write(raw)
    elif what == "medoid":
        raw = bytearray(open(g1, "rb").read())
        raw[12:16] = struct.pack("<I", shards[1][0].size)
        open(g1, "wb").write(raw)
    elif what == "truncated":
        raw = open(g1, "rb").read()
        open(g1, "wb").write(raw[:-4])
    elif what == "bad_local":
        raw = bytearray(open(g1, "rb").read())
        off = 24
        while struct.unpack_from("<I", raw, off)[0] == 0:
            off += 4
        raw[off + 4:off + 8] = struct.pack("<I", shards[1][0].size)
        open(g1, "wb").write(raw)
    return pre


ERRORS = [("missing_idmap", -2), ("idmap_dim", -2), ("idmap_size", -2), ("missing_graph", -3), ("frozen", -3),
          ("medoid", -4), ("truncated", -6), ("bad_local", -7)]


@pytest.mark.parametrize("what,code", ERRORS)
def test_oracle_error_codes(tmp_path, what, code):
    pre = corrupt(tmp_path, what)
    rc, _, _, _ = run_oracle(tmp_path, pre, 2, 8)
    assert rc == code
