"""DiskANN on-disk formats used by the builder apps.

- Matrix .bin (.fbin/.u8bin): uint32 N, uint32 dim, then N x dim row-major.
- Memory-index graph: uint64 file bytes, uint32 max degree, uint32 start
  (medoid), uint64 frozen points, then per node uint32 k and k uint32 ids
  (reference: apps/utils/gpu_vamana_memory_index.cpp:215-240).
- Ground truth: uint32 nq, uint32 k, nq*k uint32 ids, nq*k float32 distances.
- Label files: one line per point, comma-separated labels.
"""
from __future__ import annotations

import struct

import numpy as np


def write_bin(path: str, x: np.ndarray) -> None:
    x = np.ascontiguousarray(x)
    with open(path, "wb") as f:
        f.write(struct.pack("<II", x.shape[0], x.shape[1]))
        f.write(x.tobytes())


def read_bin(path: str, dtype) -> np.ndarray:
    with open(path, "rb") as f:
        n, d = struct.unpack("<II", f.read(8))
        x = np.frombuffer(f.read(), dtype=dtype)
    if x.size != n * d:
        raise ValueError(f"{path}: header {n}x{d} does not match payload")
    return x.reshape(n, d)


def read_graph(path: str):
    """Returns (adjacency list, max_degree, start, frozen)."""
    with open(path, "rb") as f:
        raw = f.read()
    total, max_deg, start, frozen = struct.unpack_from("<QIIQ", raw, 0)
    if total != len(raw):
        raise ValueError(f"{path}: header size {total} != file size {len(raw)}")
    off = 24
    adj = []
    while off < len(raw):
        (k,) = struct.unpack_from("<I", raw, off)
        off += 4
        adj.append(np.frombuffer(raw, dtype=np.uint32, count=k, offset=off).copy())
        off += 4 * k
    return adj, max_deg, start, frozen


def write_graph(path: str, graph: np.ndarray, degree: np.ndarray, start: int, R: int | None = None) -> None:
    R = graph.shape[1] if R is None else R
    deg = np.minimum(degree, R)
    body = bytearray()
    for v in range(graph.shape[0]):
        k = int(deg[v])
        body += struct.pack("<I", k) + graph[v, :k].astype(np.uint32).tobytes()
    total = 24 + len(body)
    with open(path, "wb") as f:
        f.write(struct.pack("<QIIQ", total, int(degree.max()) if degree.size else 0, start, 0))
        f.write(body)


def write_gt(path: str, ids: np.ndarray, dists: np.ndarray) -> None:
    with open(path, "wb") as f:
        f.write(struct.pack("<II", ids.shape[0], ids.shape[1]))
        f.write(np.ascontiguousarray(ids, np.uint32).tobytes())
        f.write(np.ascontiguousarray(dists, np.float32).tobytes())


def write_labels(path: str, labels: list[list[str]]) -> None:
    with open(path, "w") as f:
        for row in labels:
            f.write(",".join(row) + "\n")
