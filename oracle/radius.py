"""Brute-force radius graph oracle (C, see radius_ref.c) -- test infrastructure.

Restates src/opt_radius/mlcg_opt_radius/radius.cu:117-141 per frame, with the
canonical (i asc, j asc) order.  Pinned by:
  * scipy.spatial.cKDTree.query_ball_point set equality away from the cutoff
    boundary -- the reference's own radius test oracle
    (src/opt_radius/mlcg_opt_radius/utils.py:32-47, test_radius.py:66-104);
  * an independent numpy float32 restatement (tests/test_oracle_radius.py);
  * adversarial pairs placed exactly at d2 == fl32(r*r) and one ulp inside.
float16 / bfloat16 positions (radius_graph_narrow) follow the reference's
c10::Half / c10::BFloat16 arithmetic (every operation in float, rounded to
the 16-bit type); their conversions are pinned against numpy's float16 and
torch's bfloat16, and the search against per-operation numpy/torch
restatements (tests/test_oracle_radius.py).
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
                                            ctypes.c_int, ctypes.c_int64, P, P, P, P]
        lib.oracle_radius_count.restype = ctypes.c_int64
        lib.oracle_radius_fill.argtypes = [P, P, ctypes.c_int64, ctypes.c_double,
                                           ctypes.c_int, ctypes.c_int64, P, P, P, P]
        lib.oracle_radius_fill.restype = None
        lib.oracle_radius_count_f64.argtypes = lib.oracle_radius_count.argtypes
        lib.oracle_radius_count_f64.restype = ctypes.c_int64
        lib.oracle_radius_fill_f64.argtypes = lib.oracle_radius_fill.argtypes
        lib.oracle_radius_fill_f64.restype = None
        lib.oracle_radius_count_n16.argtypes = [ctypes.c_int] + lib.oracle_radius_count.argtypes
        lib.oracle_radius_count_n16.restype = ctypes.c_int64
        lib.oracle_radius_fill_n16.argtypes = [ctypes.c_int] + lib.oracle_radius_fill.argtypes
        lib.oracle_radius_fill_n16.restype = None
        lib.oracle_f32_to_narrow.argtypes = [ctypes.c_int, ctypes.c_float]
        lib.oracle_f32_to_narrow.restype = ctypes.c_uint16
        lib.oracle_narrow_to_f32.argtypes = [ctypes.c_int, ctypes.c_uint16]
        lib.oracle_narrow_to_f32.restype = ctypes.c_float
        _lib = lib
    return _lib


def frame_ptr_from_batch(batch: np.ndarray, n_frames: int | None = None) -> np.ndarray:
    batch = np.asarray(batch, dtype=np.int64)
    if n_frames is None:
        n_frames = int(batch[-1]) + 1 if batch.size else 0
    return np.searchsorted(batch, np.arange(n_frames + 1), side="left").astype(np.int64)


def exclusion_pair_to_ptr(exc_pair_index, num_nodes: int):
    """(pair_xs [M], y_ptr [num_nodes + 1]) restating exclusion_pairs.cpp:30-58:
    a stable lexsort by centre y (row 1), then neighbour x (row 0), and
    y_ptr[n] = number of pairs with y < n.  Raises ValueError for a negative
    y when num_nodes > 0 (the TORCH_CHECK at line 47)."""
    exc = np.asarray(exc_pair_index, dtype=np.int64).reshape(2, -1)
    x, y = exc[0], exc[1]
    order = np.lexsort((x, y))
    pair_xs = x[order]
    ys = y[order]
    if num_nodes > 0 and ys.size and ys[0] < 0:
        raise ValueError("negative centre index in the exclusion list")
    y_ptr = np.searchsorted(ys, np.arange(num_nodes + 1), side="left").astype(np.int64)
    y_ptr[0] = 0  # set unconditionally at line 42
    return pair_xs.astype(np.int64), y_ptr


def radius_graph(pos, r: float, batch=None, loop: bool = False, max_num_neighbors: int = 32,
                 n_frames: int | None = None, exclude_pair_xs=None, ptr_exclude_pair_xs=None):
    """Returns (edge_index [2, E] int64, overflow flag).  The optional
    exclusion CSR is the one exclusion_pair_to_ptr returns.  float64 positions
    are searched in double arithmetic (d2 < r*r), anything else in float32."""
    f64 = np.asarray(pos).dtype == np.float64
    pos = np.ascontiguousarray(np.asarray(pos, dtype=np.float64 if f64 else np.float32))
    n = pos.shape[0]
    if batch is None:
        batch = np.zeros(n, dtype=np.int64)
    ptr = frame_ptr_from_batch(batch, n_frames)
    nb = ptr.shape[0] - 1
    lib = _load()
    exs = eptr = None
    if exclude_pair_xs is not None:
        exs = np.ascontiguousarray(np.asarray(exclude_pair_xs, dtype=np.int64))
        if exs.size == 0:
            exs = np.zeros(1, dtype=np.int64)
        eptr = np.ascontiguousarray(np.asarray(ptr_exclude_pair_xs, dtype=np.int64))
        assert eptr.shape == (n + 1,)
    ex_p = None if exs is None else exs.ctypes.data
    ep_p = None if eptr is None else eptr.ctypes.data
    deg = np.zeros(max(n, 1), dtype=np.int64)
    ovf = ctypes.c_int(0)
    count = lib.oracle_radius_count_f64 if f64 else lib.oracle_radius_count
    fill = lib.oracle_radius_fill_f64 if f64 else lib.oracle_radius_fill
    total = count(pos.ctypes.data, ptr.ctypes.data, nb, float(r), int(loop),
                                    int(max_num_neighbors), ex_p, ep_p, deg.ctypes.data,
                                    ctypes.addressof(ovf))
    ei = np.zeros((2, max(total, 1)), dtype=np.int64)
    fill(pos.ctypes.data, ptr.ctypes.data, nb, float(r), int(loop),
                           int(max_num_neighbors), ex_p, ep_p, ei[0].ctypes.data,
                           ei[1].ctypes.data)
    return ei[:, :total].copy(), int(ovf.value)


NARROW_KINDS = {"f16": 0, "bf16": 1}


def narrow_round(kind: str, values) -> np.ndarray:
    """float32 values rounded to the 16-bit type and back (the oracle's own
    conversion, one value at a time: small arrays only)."""
    lib = _load()
    k = NARROW_KINDS[kind]
    v = np.asarray(values, dtype=np.float32).ravel()
    return np.array([lib.oracle_narrow_to_f32(k, lib.oracle_f32_to_narrow(k, float(x)))
                     for x in v], dtype=np.float32)


def radius_graph_narrow(bits, kind: str, r: float, batch=None, loop: bool = False,
                        max_num_neighbors: int = 32, n_frames: int | None = None,
                        exclude_pair_xs=None, ptr_exclude_pair_xs=None):
    """radius_graph for float16 ("f16") or bfloat16 ("bf16") positions given as
    their raw 16-bit patterns [N, 3] (uint16 / int16)."""
    k = NARROW_KINDS[kind]
    pos = np.ascontiguousarray(np.asarray(bits).view(np.uint16).reshape(-1, 3))
    n = pos.shape[0]
    if batch is None:
        batch = np.zeros(n, dtype=np.int64)
    ptr = frame_ptr_from_batch(batch, n_frames)
    nb = ptr.shape[0] - 1
    lib = _load()
    exs = eptr = None
    if exclude_pair_xs is not None:
        exs = np.ascontiguousarray(np.asarray(exclude_pair_xs, dtype=np.int64))
        if exs.size == 0:
            exs = np.zeros(1, dtype=np.int64)
        eptr = np.ascontiguousarray(np.asarray(ptr_exclude_pair_xs, dtype=np.int64))
    ex_p = None if exs is None else exs.ctypes.data
    ep_p = None if eptr is None else eptr.ctypes.data
    deg = np.zeros(max(n, 1), dtype=np.int64)
    ovf = ctypes.c_int(0)
    total = lib.oracle_radius_count_n16(k, pos.ctypes.data, ptr.ctypes.data, nb, float(r),
                                        int(loop), int(max_num_neighbors), ex_p, ep_p,
                                        deg.ctypes.data, ctypes.addressof(ovf))
    ei = np.zeros((2, max(total, 1)), dtype=np.int64)
    lib.oracle_radius_fill_n16(k, pos.ctypes.data, ptr.ctypes.data, nb, float(r), int(loop),
                               int(max_num_neighbors), ex_p, ep_p, ei[0].ctypes.data,
                               ei[1].ctypes.data)
    return ei[:, :total].copy(), int(ovf.value)
