"""Shard-graph merge: Python front-end of diskann::merge_shards_gpu.

The merge itself runs in libdance_hip.so (dance_merge_shards, the C-ABI form of
include/gpu_merge.h; reference include/gpu_merge.h:8-12, src/gpu_merge.cu:351-790).
This module only passes paths and reads the statistics; write_shard and
write_idmap produce the DiskANN files the merge consumes (shard graphs in the
memory-index format, id maps as a one-column uint32 .bin).
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np

from . import DanceMergeStats
from . import lib as _lib


def _bind():
    L = _lib()
    if not getattr(L, "_merge_bound", False):
        L.dance_merge_shards.argtypes = [C.c_char_p] * 4 + [C.c_uint64, C.c_uint32] + [C.c_char_p] * 2
        L.dance_merge_shards.restype = C.c_int
        L.dance_merge_get_last_stats.argtypes = [C.POINTER(DanceMergeStats)]
        L.dance_merge_get_last_stats.restype = None
        L._merge_bound = True
    return L


def merge_shards(vamana_prefix: str, vamana_suffix: str, idmaps_prefix: str, idmaps_suffix: str, nshards: int,
                 max_degree: int, output_vamana: str, medoids_file: str) -> int:
    """diskann::merge_shards_gpu: returns its code (0, or the reference's negative codes)."""
    L = _bind()
    return int(L.dance_merge_shards(vamana_prefix.encode(), vamana_suffix.encode(), idmaps_prefix.encode(),
                                    idmaps_suffix.encode(), nshards, max_degree, output_vamana.encode(),
                                    medoids_file.encode()))


def last_stats() -> dict:
    L = _bind()
    s = DanceMergeStats()
    L.dance_merge_get_last_stats(C.byref(s))
    return {name: getattr(s, name) for name, _ in DanceMergeStats._fields_ if not name.startswith("reserved")}


def write_idmap(path: str, ids) -> None:
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    with open(path, "wb") as f:
        f.write(struct.pack("<II", ids.size, 1))
        f.write(ids.tobytes())


def write_shard(path: str, adjacency, medoid: int, width: int | None = None, frozen: int = 0) -> None:
    """A DiskANN memory-index graph from per-node neighbour lists (local ids)."""
    rows = [np.ascontiguousarray(a, dtype=np.uint32) for a in adjacency]
    width = max((r.size for r in rows), default=0) if width is None else width
    body = b"".join(struct.pack("<I", r.size) + r.tobytes() for r in rows)
    with open(path, "wb") as f:
        f.write(struct.pack("<QIIQ", 24 + len(body), width, medoid, frozen))
        f.write(body)
