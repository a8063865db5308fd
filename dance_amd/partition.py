"""Shard assignment of the sharded build: Python front-end of
dance_partition_assign (libdance_hip.so).

Each row's k_base nearest centers under squared L2 accumulated in fp64 in
dimension order, ties to the lower center index (DiskANN's
shard_data_into_clusters_only_ids, called from build_merged_vamana_index,
reference integrations/dance-diskann-78256bba.patch:1212-1260). The full
pipeline (sample, k-means, per-shard GPU builds, merge) is the
build_sharded_index app.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import DTYPE_F32, DTYPE_U8
from . import lib as _lib


def _bind():
    L = _lib()
    if not getattr(L, "_partition_bound", False):
        L.dance_partition_assign.argtypes = [C.c_void_p, C.c_int, C.c_uint64, C.c_uint32, C.POINTER(C.c_float),
                                             C.c_uint32, C.c_uint32, C.POINTER(C.c_uint32)]
        L.dance_partition_assign.restype = C.c_int
        L._partition_bound = True
    return L


def assign_rc(data: np.ndarray, centers: np.ndarray, k_base: int, out: np.ndarray | None = None) -> tuple[int, np.ndarray]:
    """Calls the C ABI; returns (code, N x k_base uint32)."""
    data = np.ascontiguousarray(data)
    centers = np.ascontiguousarray(centers, np.float32)
    if data.dtype == np.float32:
        dt = DTYPE_F32
    elif data.dtype == np.uint8:
        dt = DTYPE_U8
    else:
        raise TypeError("rows must be float32 or uint8")
    out = np.empty((data.shape[0], max(k_base, 1)), np.uint32) if out is None else out
    rc = _bind().dance_partition_assign(data.ctypes.data, dt, data.shape[0], data.shape[1],
                                        centers.ctypes.data_as(C.POINTER(C.c_float)), centers.shape[0], k_base,
                                        out.ctypes.data_as(C.POINTER(C.c_uint32)))
    return int(rc), out


def assign(data: np.ndarray, centers: np.ndarray, k_base: int) -> np.ndarray:
    rc, out = assign_rc(data, centers, k_base)
    if rc != 0:
        raise RuntimeError(f"dance_partition_assign returned {rc}")
    return out
