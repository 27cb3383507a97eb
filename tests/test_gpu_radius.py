"""HIP radius graph against the C oracle: bit-exact edge lists.

Parameter sweep mirrors src/opt_radius/mlcg_opt_radius/test_radius.py:31-104
(node counts 0/10/100, two coordinate ranges, r in {0, 1, 10}, one to three
frames, loop on and off) restricted to 3-D positions; plus the full config-3
workload and adversarial boundary pairs.
"""

import math
from itertools import product

import numpy as np
import pytest
import torch

from oracle import radius as oracle_radius

pytestmark = pytest.mark.gpu

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


def _hip(pos, r, batch, loop, mnn, with_pairs=False):
    from mlcg_amd import ops

    g = ops.radius_graph(torch.from_numpy(pos).cuda(), r,
                         batch=torch.from_numpy(batch).cuda(), loop=loop,
                         max_num_neighbors=mnn, with_pairs=with_pairs,
                         n_frames=int(batch.max()) + 1 if batch.size else 0)
    return g


@pytest.mark.parametrize("n,x_range,r,split,loop", list(product(X, X_RANGE, R, BATCH_SIZES, LOOP)))
def test_radius_sweep(n, x_range, r, split, loop):
    rng = np.random.default_rng(1000 + n)
    lo, hi = x_range
    pos = ((hi - lo) * rng.random((n, 3)) + lo).astype(np.float32)
    batch = _batch(n, split)
    ref, _ = oracle_radius.radius_graph(pos, r, batch, loop, 100)
    g = _hip(pos, r, batch, loop, 100)
    got = g.edge_index.cpu().numpy()
    assert got.shape == ref.shape
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("mnn", [1, 3, 7])
def test_radius_max_num_neighbors(mnn):
    """Binding cap keeps the lowest-index neighbours (radius.cu:125-141)."""
    rng = np.random.default_rng(7)
    pos = (rng.random((150, 3)) * 4).astype(np.float32)
    batch = _batch(150, (40, 100))
    ref, ovf = oracle_radius.radius_graph(pos, 2.0, batch, False, mnn)
    assert ovf == 1
    g = _hip(pos, 2.0, batch, False, mnn)
    assert g.overflow & 1
    assert np.array_equal(g.edge_index.cpu().numpy(), ref)


def test_radius_boundary_exact():
    """A pair exactly at d2 == fl32(r^2) is excluded (strict <), one a float
    ulp closer is included; the same holds for off-axis pairs whose fp32 d2
    rounds onto the boundary."""
    r = 15.0
    x_in = float(np.nextafter(np.float32(15.0), np.float32(0.0)))
    pos = np.array([[0, 0, 0], [15.0, 0, 0],            # frame 0: d2 == 225, out
                    [0, 0, 0], [x_in, 0, 0],            # frame 1: just inside
                    [1, 2, 3], [10.0, 14.0, 5.0],       # frame 2: generic
                    [0, 0, 0], [9.0, 12.0, 0.0]],       # frame 3: 81+144 == 225, out
                   dtype=np.float32)
    batch = np.array([0, 0, 1, 1, 2, 2, 3, 3], dtype=np.int64)
    ref, _ = oracle_radius.radius_graph(pos, r, batch, False, 32)
    assert ref.tolist() == [[2, 3], [3, 2]]
    g = _hip(pos, r, batch, False, 32)
    assert np.array_equal(g.edge_index.cpu().numpy(), ref)


def test_radius_config3_bit_exact():
    from mlcg_amd import synthetic

    b = synthetic.config3()
    ref, _ = oracle_radius.radius_graph(b.pos, 15.0, b.batch, False, 1000)
    g = _hip(b.pos, 15.0, b.batch, False, 1000)
    got = g.edge_index.cpu().numpy()
    print(f"config3: N={b.pos.shape[0]} E={ref.shape[1]}")
    assert got.shape == ref.shape
    assert np.array_equal(got, ref)


def test_pair_structures():
    """pair_ij = upper edges in order; eid2pair maps both copies of a pair."""
    from mlcg_amd import synthetic

    b = synthetic.config2(n_frames=16)
    g = _hip(b.pos, 20.0, b.batch, False, 1000, with_pairs=True)
    ei = g.edge_index.cpu().numpy()
    pij = g.pair_ij.cpu().numpy()
    e2p = g.eid2pair.cpu().numpy()
    up = ei[0] < ei[1]
    assert np.array_equal(pij, ei[:, up].astype(np.int32))
    assert g.num_pairs * 2 == g.num_edges
    pi, pj = pij[0][e2p], pij[1][e2p]
    assert np.array_equal(np.minimum(ei[0], ei[1]), pi)
    assert np.array_equal(np.maximum(ei[0], ei[1]), pj)
    rowptr = g.rowptr.cpu().numpy()
    assert np.array_equal(np.diff(rowptr), np.bincount(ei[0], minlength=b.pos.shape[0]))
    assert np.array_equal(g.col.cpu().numpy(), ei[1].astype(np.int32))


def test_radius_deterministic():
    from mlcg_amd import synthetic

    b = synthetic.config2(n_frames=64)
    g1 = _hip(b.pos, 20.0, b.batch, False, 1000, with_pairs=True)
    g2 = _hip(b.pos, 20.0, b.batch, False, 1000, with_pairs=True)
    assert torch.equal(g1.edge_index, g2.edge_index)
    assert torch.equal(g1.eid2pair, g2.eid2pair)
