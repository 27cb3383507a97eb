"""Pins the C radius-graph oracle (oracle/radius_ref.c) without a GPU.

What pins it:
  * the reference's own radius test sweep (src/opt_radius/mlcg_opt_radius/
    test_radius.py:31-104: N in {0, 10, 100}, two coordinate ranges,
    r in {0, 1, 10}, 1-3 frames, loop on/off) against
    scipy.spatial.cKDTree.query_ball_point -- the reference's kd-tree oracle
    (utils.py:32-47) -- as set equality, with pairs within 1e-4 A of the
    cutoff excluded from the comparison (the kd-tree works in float64);
  * exact boundary cases: d2 == fl32(r^2) is outside (strict `<`,
    radius.cu:134), one float ulp closer is inside, and an off-axis pair whose
    fp32 d2 rounds onto the boundary;
  * the max_num_neighbors cap keeps the lowest-index neighbours
    (radius.cu:125-141), checked against a sort of the kd-tree hits;
  * the canonical order (rows ascending, neighbours ascending), frames never
    mixed, no self loops unless asked.
"""

import math
from itertools import product

import numpy as np
import pytest
from scipy.spatial import cKDTree

from oracle import radius as oracle_radius

X = [0, 10, 100]
X_RANGE = [(-1.0, 1.0), (-10.0, -20.0)]
R = [0.0, 1.0, 10.0]
BATCH_SIZES = [(100,), (50, 100), (10, 20, 100)]
LOOP = [True, False]


def _batch(n, split):
    out, p = [], 0
    for i, b in enumerate(split):
        k = math.ceil(n * (b / 100)) - p
        out.append(np.full(k, i, dtype=np.int64))
        p += k
    return np.concatenate(out) if out else np.zeros(0, np.int64)


def _kdtree_pairs(pos, r, batch, loop):
    """Set of (i, j) from per-frame kd-trees, plus the set of pairs whose
    float64 distance is within 1e-4 of r (ambiguous for the fp32 test)."""
    pairs, near = set(), set()
    pos64 = pos.astype(np.float64)
    for b in np.unique(batch):
        idx = np.nonzero(batch == b)[0]
        tree = cKDTree(pos64[idx])
        for a, hits in enumerate(tree.query_ball_point(pos64[idx], r + 1e-4)):
            for h in hits:
                i, j = int(idx[a]), int(idx[h])
                if i == j and not loop:
                    continue
                d = np.linalg.norm(pos64[j] - pos64[i])
                if abs(d - r) <= 1e-4:
                    near.add((i, j))
                elif d < r:
                    pairs.add((i, j))
    return pairs, near


@pytest.mark.parametrize("n,x_range,r,split,loop",
                         list(product(X, X_RANGE, R, BATCH_SIZES, LOOP)))
def test_oracle_vs_kdtree_sweep(n, x_range, r, split, loop):
    rng = np.random.default_rng(1000 + n)
    lo, hi = x_range
    pos = ((hi - lo) * rng.random((n, 3)) + lo).astype(np.float32)
    batch = _batch(n, split)
    ei, ovf = oracle_radius.radius_graph(pos, r, batch, loop, 1000)
    assert ovf == 0
    got = set(map(tuple, ei.T.tolist()))
    want, near = _kdtree_pairs(pos, r, batch, loop)
    assert got - near == want - near
    # canonical order, frames not mixed, self loops only with loop=True
    if ei.shape[1]:
        key = ei[0] * (n + 1) + ei[1]
        assert np.all(np.diff(key) > 0)
        assert np.array_equal(batch[ei[0]], batch[ei[1]])
        assert loop or np.all(ei[0] != ei[1])


def test_oracle_boundary_exact():
    r = 15.0
    x_in = float(np.nextafter(np.float32(15.0), np.float32(0.0)))
    pos = np.array([[0, 0, 0], [15.0, 0, 0],
                    [0, 0, 0], [x_in, 0, 0],
                    [0, 0, 0], [9.0, 12.0, 0.0],
                    [1, 2, 3], [10.0, 14.0, 5.0]], dtype=np.float32)
    batch = np.array([0, 0, 1, 1, 2, 2, 3, 3], dtype=np.int64)
    ei, _ = oracle_radius.radius_graph(pos, r, batch, False, 32)
    assert ei.tolist() == [[2, 3], [3, 2]]
    # with the cutoff a hair larger the boundary pairs join
    ei2, _ = oracle_radius.radius_graph(pos, 15.0001, batch, False, 32)
    assert sorted(map(tuple, ei2.T.tolist())) == [(0, 1), (1, 0), (2, 3), (3, 2), (4, 5),
                                                  (5, 4)]


def test_oracle_r2_rounding_of_cutoff():
    """r^2 is formed in double and rounded once to fp32 (radius.cu:250): a
    pair with fp32 d2 equal to fl32(r*r) stays outside even when r*r is not
    representable."""
    r = 0.1
    r2 = np.float32(r * r)
    # construct dx with fl32(dx*dx) == r2 exactly if possible, else closest below
    dx = np.float32(np.sqrt(np.float64(r2)))
    while np.float32(dx * dx) > r2:
        dx = np.nextafter(dx, np.float32(0))
    pos = np.array([[0, 0, 0], [dx, 0, 0]], dtype=np.float32)
    ei, _ = oracle_radius.radius_graph(pos, r, None, False, 8)
    inside = np.float32(dx * dx) < r2
    assert (ei.shape[1] == 2) == bool(inside)


@pytest.mark.parametrize("mnn", [1, 3, 7])
def test_oracle_max_num_neighbors(mnn):
    rng = np.random.default_rng(7)
    pos = (rng.random((150, 3)) * 4).astype(np.float32)
    batch = _batch(150, (40, 100))
    ei, ovf = oracle_radius.radius_graph(pos, 2.0, batch, False, mnn)
    assert ovf == 1
    full, _ = oracle_radius.radius_graph(pos, 2.0, batch, False, 10_000)
    # every row keeps exactly its min(mnn, deg) lowest-index neighbours
    for i in range(150):
        row_full = full[1][full[0] == i]
        row = ei[1][ei[0] == i]
        assert np.array_equal(row, np.sort(row_full)[:mnn])


def test_oracle_empty_and_single():
    ei, _ = oracle_radius.radius_graph(np.zeros((0, 3), np.float32), 1.0, None, False, 8)
    assert ei.shape == (2, 0)
    ei, _ = oracle_radius.radius_graph(np.zeros((1, 3), np.float32), 1.0, None, False, 8)
    assert ei.shape == (2, 0)
    ei, _ = oracle_radius.radius_graph(np.zeros((1, 3), np.float32), 1.0, None, True, 8)
    assert ei.tolist() == [[0], [0]]


def test_oracle_golden_fixture():
    """Committed fixture (tests/golden/make_golden.py) of a small config-3-like
    batch: the oracle must keep producing exactly these edges."""
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", "radius_small.npz")
    g = np.load(path)
    ei, _ = oracle_radius.radius_graph(g["pos"], float(g["r"]), g["batch"], False, 1000)
    assert np.array_equal(ei, g["edge_index"])


# ---------------------------------------------------------------------------
# Pair exclusion (radius.cu:113-133, exclusion_pairs.cpp:7-62)

def test_exclusion_to_ptr_worked_example():
    """Pairs (x, y) = (2,1), (1,2), (3,2), (2,2), (2,3), num_nodes = 4.
    Following the code of exclusion_pairs.cpp:30-58 by hand (stable argsort
    by x, then stable argsort by y; y_ptr[n+1] = pairs with y <= n): the
    y = 1 row holds x = 2, the y = 2 row x = 1, 2, 3, the y = 3 row x = 2.
    (The comment example at exclusion_pairs.cpp:15-19 lists other values;
    the code is what the kernel consumes.)"""
    exc = np.array([[2, 1, 3, 2, 2], [1, 2, 2, 2, 3]], dtype=np.int64)
    xs, yp = oracle_radius.exclusion_pair_to_ptr(exc, 4)
    assert xs.tolist() == [2, 1, 2, 3, 2]
    assert yp.tolist() == [0, 0, 1, 4, 5]


def _random_exclusions(rng, n, m, n_out=0):
    x = rng.integers(0, max(n, 1), m)
    y = rng.integers(0, max(n, 1), m)
    if n_out:  # centres past the last node stay outside every row
        x = np.concatenate([x, rng.integers(0, n, n_out)])
        y = np.concatenate([y, rng.integers(n, n + 5, n_out)])
    return np.stack([x, y]).astype(np.int64)


def test_exclusion_to_ptr_rows_brute_force():
    rng = np.random.default_rng(11)
    n = 40
    exc = _random_exclusions(rng, n, 300, n_out=7)  # includes duplicates
    xs, yp = oracle_radius.exclusion_pair_to_ptr(exc, n)
    assert yp.shape == (n + 1,) and yp[0] == 0 and yp[-1] == 300
    assert xs.shape == (307,)
    for y in range(n):
        seg = xs[yp[y]:yp[y + 1]]
        want = np.sort(exc[0][exc[1] == y])
        assert np.array_equal(seg, want)
    # the 7 out-of-range centres come last, ordered by (y, x)
    tail = sorted(zip(exc[1][300:], exc[0][300:]))
    assert xs[300:].tolist() == [x for _, x in tail]


def test_exclusion_to_ptr_negative_centre():
    exc = np.array([[0, 1], [-1, 0]], dtype=np.int64)
    with pytest.raises(ValueError):
        oracle_radius.exclusion_pair_to_ptr(exc, 3)
    xs, yp = oracle_radius.exclusion_pair_to_ptr(exc, 0)  # no rows: nothing checked
    assert yp.tolist() == [0] and xs.tolist() == [0, 1]


def _brute_rows(pos, r, batch, loop, mnn, excluded):
    """Independent numpy float32 restatement: per row, candidates ascending,
    drop excluded (i, j), keep the first mnn hits."""
    r2 = np.float32(r * r)
    out = []
    for i in range(pos.shape[0]):
        kept = 0
        for j in np.nonzero(batch == batch[i])[0]:
            if (j == i and not loop) or (i, int(j)) in excluded:
                continue
            d = pos[j] - pos[i]
            s = np.float32(d[0] * d[0])
            s = np.float32(s + np.float32(d[1] * d[1]))
            s = np.float32(s + np.float32(d[2] * d[2]))
            if s < r2 and kept < mnn:
                out.append((i, int(j)))
                kept += 1
    return np.array(out, dtype=np.int64).reshape(-1, 2).T


@pytest.mark.parametrize("loop,mnn", [(False, 1000), (True, 1000), (False, 3)])
def test_oracle_exclusions_brute_force(loop, mnn):
    """Exclusion = set difference on the edge (y, x) of every pair (x, y),
    self pairs included, cross-frame pairs and duplicates harmless, and
    excluded neighbours not counted towards max_num_neighbors."""
    rng = np.random.default_rng(5 + mnn + int(loop))
    n = 90
    pos = (rng.random((n, 3)) * 5).astype(np.float32)
    batch = _batch(n, (30, 70, 100))
    exc = _random_exclusions(rng, n, 600)
    exc = np.concatenate([exc, np.stack([np.arange(0, n, 7)] * 2)], axis=1)  # self pairs
    xs, yp = oracle_radius.exclusion_pair_to_ptr(exc, n)
    ei, _ = oracle_radius.radius_graph(pos, 2.5, batch, loop, mnn, exclude_pair_xs=xs,
                                       ptr_exclude_pair_xs=yp)
    excluded = set(zip(exc[1].tolist(), exc[0].tolist()))
    want = _brute_rows(pos, 2.5, batch, loop, mnn, excluded)
    assert np.array_equal(ei, want)
    full, _ = oracle_radius.radius_graph(pos, 2.5, batch, loop, mnn)
    if mnn >= n:
        diff = {e for e in zip(*full.tolist())} - excluded
        assert set(zip(*ei.tolist())) == diff
        assert ei.shape[1] < full.shape[1]


def test_oracle_exclusions_empty_list():
    rng = np.random.default_rng(3)
    pos = (rng.random((30, 3)) * 3).astype(np.float32)
    xs, yp = oracle_radius.exclusion_pair_to_ptr(np.zeros((2, 0), np.int64), 30)
    ei, _ = oracle_radius.radius_graph(pos, 1.5, None, False, 100, exclude_pair_xs=xs,
                                       ptr_exclude_pair_xs=yp)
    full, _ = oracle_radius.radius_graph(pos, 1.5, None, False, 100)
    assert np.array_equal(ei, full)


@pytest.mark.parametrize("n,x_range,r,split,loop",
                         list(product(X, X_RANGE, R, BATCH_SIZES, LOOP)))
def test_oracle_f64_vs_kdtree_sweep(n, x_range, r, split, loop):
    """float64 positions: the double-arithmetic search against scipy's kd-tree
    away from the boundary (the sweep of test_radius.py:66-104, which runs the
    reference's kernel in float64)."""
    rng = np.random.default_rng(2000 + n)
    lo, hi = x_range
    pos = (hi - lo) * rng.random((n, 3)) + lo
    batch = _batch(n, split)
    ei, ovf = oracle_radius.radius_graph(pos, r, batch, loop, 1000)
    assert ovf == 0
    got = set(map(tuple, ei.T.tolist()))
    want, near = _kdtree_pairs(pos, r, batch, loop)
    assert got - near == want - near


def test_oracle_f64_boundary_is_decided_in_double():
    """A pair whose float64 d2 lies one double ulp below r*r is inside in
    double arithmetic although its float32 rounding sits on the cutoff: the
    float64 search does not round positions to float32 first.  Also: a pair at
    exactly d2 == r*r stays outside (strict <)."""
    r = 1.0
    x = float(np.nextafter(1.0, 0.0))  # x*x < 1 in double; float32(x) == 1.0
    assert np.float32(x) == np.float32(1.0) and x * x < 1.0
    pos = np.array([[0.0, 0, 0], [x, 0, 0], [0.0, 0, 0], [1.0, 0, 0]])
    batch = np.array([0, 0, 1, 1])
    ei, _ = oracle_radius.radius_graph(pos, r, batch, False, 8)
    assert ei.tolist() == [[0, 1], [1, 0]]
    ei32, _ = oracle_radius.radius_graph(pos.astype(np.float32), r, batch, False, 8)
    assert ei32.shape[1] == 0


def test_oracle_f64_numpy_restatement():
    """The double search equals a plain numpy double restatement (d2 summed
    as ((dx^2 + dy^2) + dz^2), strict < r*r) on random frames."""
    rng = np.random.default_rng(17)
    pos = rng.random((90, 3)) * 3.0
    batch = np.repeat(np.arange(3), 30)
    r = 0.9
    ei, _ = oracle_radius.radius_graph(pos, r, batch, False, 1000)
    want = []
    for i in range(90):
        for j in range(90):
            if i == j or batch[i] != batch[j]:
                continue
            d = pos[j] - pos[i]
            if (d[0] * d[0] + d[1] * d[1]) + d[2] * d[2] < r * r:
                want.append((i, j))
    assert list(map(tuple, ei.T.tolist())) == want


# --------------------------------------------------------------------------
# float16 / bfloat16 positions (the reference's Half / BFloat16 dispatch,
# radius.cu:243-250): c10 scalar arithmetic, every operation in float and
# rounded to the 16-bit type.

def test_oracle_f16_conversions_match_numpy():
    """All 2^16 binary16 patterns widen like numpy's float16, and float32
    values (random, exact ties, subnormal range, overflow) round like numpy's
    float32 -> float16 cast (round to nearest even)."""
    lib = oracle_radius._load()
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.oracle_narrow_to_f32(0, int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    rng = np.random.default_rng(3)
    h = rng.integers(0, 0x7c00, 4000, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float32)
    hi = (h + 1).view(np.float16).astype(np.float32)
    ties = (lo.astype(np.float64) + hi.astype(np.float64)) / 2  # exact in float32
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-9, 5, 4000),
        ties.astype(np.float32), -ties.astype(np.float32),
        np.float32([0.0, -0.0, 65504.0, 65519.99, 65520.0, 7e4, 5.96e-8, 2.98e-8, 3e-8,
                    6.1e-5, 6.09e-5, np.inf, -np.inf])])
    got = np.array([lib.oracle_f32_to_narrow(0, float(v)) for v in vals], dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_oracle_bf16_conversions_match_torch():
    """bfloat16 widening is exact and the float32 -> bfloat16 rounding equals
    torch's (round to nearest even), ties included."""
    import torch

    lib = oracle_radius._load()
    rng = np.random.default_rng(4)
    b = rng.integers(0, 0x7f80, 3000, dtype=np.uint16)
    wide = (b.astype(np.uint32) << 16).view(np.float32)
    got = np.array([lib.oracle_narrow_to_f32(1, int(x)) for x in b], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), wide.view(np.uint32))
    nxt = ((b.astype(np.uint32) + 1) << 16).view(np.float32)
    ties = ((wide.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    vals = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 100.0, ties, -ties,
                           np.float32([0.0, -0.0, 3.4e38, np.inf, -np.inf])])
    got = np.array([lib.oracle_f32_to_narrow(1, float(v)) for v in vals], dtype=np.uint16)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def _narrow_restatement(d16, r, batch, loop):
    """Edges of a per-operation 16-bit restatement: d16 computes (x_j - x_i)
    squared and summed ((dx^2 + dy^2) + dz^2) in the 16-bit type, r2 is the
    16-bit rounding of float32(r*r)."""
    n = batch.shape[0]
    want = []
    for i in range(n):
        d2, r2 = d16(i)
        for j in range(n):
            if batch[i] != batch[j] or (not loop and i == j):
                continue
            if d2[j] < r2:
                want.append((i, j))
    return want


def test_oracle_f16_search_matches_numpy_float16():
    """The float16 search equals numpy float16 arithmetic (numpy computes each
    float16 operation in float32 and rounds, the c10 semantics) on random
    frames, including self loops and a max_num_neighbors cap."""
    rng = np.random.default_rng(21)
    pos = (rng.random((80, 3)) * 6.0).astype(np.float16)
    batch = np.repeat(np.arange(2), 40)
    r = 2.1
    r2 = np.float16(np.float32(r * r))

    def d16(i):
        d = pos - pos[i]  # float16 (x_j - x_i)
        sq = d * d
        return (sq[:, 0] + sq[:, 1]) + sq[:, 2], r2

    for loop in (False, True):
        ei, _ = oracle_radius.radius_graph_narrow(pos.view(np.uint16), "f16", r, batch, loop,
                                                  1000)
        assert list(map(tuple, ei.T.tolist())) == _narrow_restatement(d16, r, batch, loop)
    ei, ovf = oracle_radius.radius_graph_narrow(pos.view(np.uint16), "f16", r, batch, False, 3)
    full = _narrow_restatement(d16, r, batch, False)
    capped = [e for e in full if sum(1 for f in full if f[0] == e[0] and f[1] <= e[1]) <= 3]
    assert list(map(tuple, ei.T.tolist())) == capped and ovf == 1


def test_oracle_bf16_search_matches_torch_bfloat16():
    """The bfloat16 search equals torch's CPU bfloat16 arithmetic (each
    operation in float, rounded to bfloat16) on random frames."""
    import torch

    rng = np.random.default_rng(22)
    pos = torch.from_numpy(rng.random((70, 3)).astype(np.float32) * 6.0).to(torch.bfloat16)
    batch = np.repeat(np.arange(2), 35)
    r = 2.3
    r2 = torch.tensor(np.float32(r * r)).to(torch.bfloat16).float().item()

    def d16(i):
        d = pos - pos[i]
        sq = d * d
        return ((sq[:, 0] + sq[:, 1]) + sq[:, 2]).float().numpy(), r2

    bits = pos.view(torch.int16).numpy().view(np.uint16)
    ei, _ = oracle_radius.radius_graph_narrow(bits, "bf16", r, batch, False, 1000)
    assert list(map(tuple, ei.T.tolist())) == _narrow_restatement(d16, r, batch, False)


def test_oracle_f16_boundary_in_half_precision():
    """A pair whose float16 d2 equals the float16 r2 is outside (strict <);
    moved one float16 ulp closer it is inside; a pair inside in float32 but
    rounded onto r2 by the float16 subtraction is outside."""
    r = 1.5
    r2 = np.float16(np.float32(r * r))  # 2.25 exactly
    x = np.float16(1.5)
    pos = np.array([[0, 0, 0], [x, 0, 0]], dtype=np.float16)
    ei, _ = oracle_radius.radius_graph_narrow(pos.view(np.uint16), "f16", r)
    assert ei.shape[1] == 0 and float(np.float16(x * x)) == float(r2)
    closer = np.nextafter(x, np.float16(0))
    pos[1, 0] = closer
    ei, _ = oracle_radius.radius_graph_narrow(pos.view(np.uint16), "f16", r)
    assert ei.T.tolist() == [[0, 1], [1, 0]]
    # exact difference 1.5 - 1e-4 (inside in float32) rounds to 1.5 in the
    # float16 subtraction, so d2 lands on r2: outside
    a, b = np.float16(1e-4), np.float16(1.5)
    assert (np.float32(b) - np.float32(a)) ** 2 < np.float32(r * r)
    assert b - a == np.float16(1.5)
    pos = np.array([[a, 0, 0], [b, 0, 0]], dtype=np.float16)
    ei, _ = oracle_radius.radius_graph_narrow(pos.view(np.uint16), "f16", r)
    assert ei.shape[1] == 0
