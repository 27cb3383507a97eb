"""Brute-force radius graph oracle (C, see radius_ref.c) -- test infrastructure.

Restates src/opt_radius/mlcg_opt_radius/radius.cu:117-141 per frame, with the
canonical (i asc, j asc) order.  Pinned by:
  * scipy.spatial.cKDTree.query_ball_point set equality away from the cutoff
    boundary -- the reference's own radius test oracle
    (src/opt_radius/mlcg_opt_radius/utils.py:32-47, test_radius.py:66-104);
  * an independent numpy float32 restatement (tests/test_oracle_radius.py);
  * adversarial pairs placed exactly at d2 == fl32(r*r) and one ulp inside.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle_radius.so")
_lib = None


def build() -> str:
    subprocess.check_call(["make", "-s", "-C", _HERE], stdout=subprocess.DEVNULL)
    return _SO


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        lib = ctypes.CDLL(_SO)
        P = ctypes.c_void_p
        lib.oracle_radius_count.argtypes = [P, P, ctypes.c_int64, ctypes.c_double,
                                            ctypes.c_int, ctypes.c_int64, P, P]
        lib.oracle_radius_count.restype = ctypes.c_int64
        lib.oracle_radius_fill.argtypes = [P, P, ctypes.c_int64, ctypes.c_double,
                                           ctypes.c_int, ctypes.c_int64, P, P]
        lib.oracle_radius_fill.restype = None
        _lib = lib
    return _lib


def frame_ptr_from_batch(batch: np.ndarray, n_frames: int | None = None) -> np.ndarray:
    batch = np.asarray(batch, dtype=np.int64)
    if n_frames is None:
        n_frames = int(batch[-1]) + 1 if batch.size else 0
    return np.searchsorted(batch, np.arange(n_frames + 1), side="left").astype(np.int64)


def radius_graph(pos, r: float, batch=None, loop: bool = False, max_num_neighbors: int = 32,
                 n_frames: int | None = None):
    """Returns (edge_index [2, E] int64, overflow flag)."""
    pos = np.ascontiguousarray(np.asarray(pos, dtype=np.float32))
    n = pos.shape[0]
    if batch is None:
        batch = np.zeros(n, dtype=np.int64)
    ptr = frame_ptr_from_batch(batch, n_frames)
    nb = ptr.shape[0] - 1
    lib = _load()
    deg = np.zeros(max(n, 1), dtype=np.int64)
    ovf = ctypes.c_int(0)
    total = lib.oracle_radius_count(pos.ctypes.data, ptr.ctypes.data, nb, float(r), int(loop),
                                    int(max_num_neighbors), deg.ctypes.data,
                                    ctypes.addressof(ovf))
    ei = np.zeros((2, max(total, 1)), dtype=np.int64)
    lib.oracle_radius_fill(pos.ctypes.data, ptr.ctypes.data, nb, float(r), int(loop),
                           int(max_num_neighbors), ei[0].ctypes.data, ei[1].ctypes.data)
    return ei[:, :total].copy(), int(ovf.value)
