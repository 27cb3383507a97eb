"""The radius graph's row-block kernel in its three modes -- the sizing pass
(mlcg_radius_rowptr: counts, block scan, decoupled look-back), the write pass
given the CSR (mlcg_radius_fill) and the one-launch fixed-capacity form
(mlcg_radius_graph) -- against the C oracle, bit for bit.

The cases reach every path of the kernel: frames staged in LDS and frames too
large to stage, rows whose hit masks are kept (up to 512 candidates) and
longer rows that are tested again in the write pass, from LDS or from global
memory, blocks that span many small frames, more than 256 predecessors in the
look-back (config 3 has 1,024 blocks of 200 rows), a binding
max_num_neighbors, self loops, pair exclusions, float64 positions, a
capacity that is too small, an empty input and one workspace reused by calls
of different sizes.  The reference's own sweep (test_radius.py:31-104) stops
at 100 nodes; the larger cases here follow its construction (uniform
positions, frames by percentage split)."""

import numpy as np
import pytest
import torch

from oracle import radius as oracle_radius

pytestmark = pytest.mark.gpu


def _frames(sizes):
    return np.repeat(np.arange(len(sizes)), sizes).astype(np.int64)


def _case(name):
    rng = np.random.default_rng({"config3": 0, "long_rows": 1, "huge_frame": 2, "ragged": 3,
                                 "mid_rows": 4}[name])
    if name == "config3":
        from mlcg_amd import synthetic

        b = synthetic.config3()
        return b.pos, b.batch, 15.0
    if name == "long_rows":  # 18 chunks per row: masks overflow, staged and unstaged blocks
        sizes = [1100, 1100, 1100]
        pos = (rng.random((sum(sizes), 3)) * 25.0).astype(np.float32)
        return pos, _frames(sizes), 12.0
    if name == "mid_rows":  # 11 chunks per row, blocks inside one frame staged
        sizes = [700] * 4
        pos = (rng.random((sum(sizes), 3)) * 22.0).astype(np.float32)
        return pos, _frames(sizes), 10.0
    if name == "huge_frame":  # 2500-node frame: never staged
        pos = (rng.random((2500, 3)) * 30.0).astype(np.float32)
        return pos, _frames([2500]), 9.0
    if name == "ragged":  # many small frames per block, some empty of neighbours
        sizes = rng.integers(1, 300, 60)
        pos = (rng.random((int(sizes.sum()), 3)) * 20.0).astype(np.float32)
        return pos, _frames(sizes), 4.0
    raise ValueError(name)


def _graph(pos, batch, r, loop, mnn, **kw):
    from mlcg_amd import ops

    nf = int(batch.max()) + 1 if batch.size else 0
    return ops.radius_graph(torch.from_numpy(pos).cuda(), r,
                            batch=torch.from_numpy(batch).cuda(), loop=loop,
                            max_num_neighbors=mnn, n_frames=nf, **kw)


def _rowptr_ref(ei, n):
    return np.concatenate([[0], np.cumsum(np.bincount(ei[0], minlength=n))]).astype(np.int32)


@pytest.mark.parametrize("name,loop,mnn", [("config3", False, 1000), ("long_rows", False, 10 ** 6),
                                           ("long_rows", True, 1500), ("huge_frame", False, 7),
                                           ("mid_rows", False, 10 ** 6), ("mid_rows", True, 90),
                                           ("ragged", True, 1000), ("ragged", False, 3)])
def test_exact_and_capacity_forms(name, loop, mnn):
    pos, batch, r = _case(name)
    n = pos.shape[0]
    print(f"case {name} n={n} loop={loop} mnn={mnn}", flush=True)
    ref, ovf = oracle_radius.radius_graph(pos, r, batch, loop, mnn)
    E = ref.shape[1]
    g = _graph(pos, batch, r, loop, mnn)
    assert np.array_equal(g.edge_index.cpu().numpy(), ref)
    assert np.array_equal(g.rowptr.cpu().numpy(), _rowptr_ref(ref, n))
    gc = _graph(pos, batch, r, loop, mnn, capacity=E + 100)
    flags = int(gc.flags.item())
    assert flags & ~1 == 0 and bool(flags & 1) == bool(ovf)
    assert np.array_equal(gc.edge_index[:, :E].cpu().numpy(), ref)
    assert np.array_equal(gc.rowptr.cpu().numpy(), _rowptr_ref(ref, n))


@pytest.mark.parametrize("name", ["config3", "long_rows", "huge_frame", "mid_rows"])
def test_pair_structures_both_forms(name):
    """col, pair_ij, pairptr and eid2pair from the fused form equal the
    exactly-sized graph's, and the exact ones follow from the edge list."""
    pos, batch, r = _case(name)
    n = pos.shape[0]
    g = _graph(pos, batch, r, False, 10 ** 6, with_pairs=True)
    ei = g.edge_index.cpu().numpy()
    up = ei[0] < ei[1]
    assert np.array_equal(g.pair_ij.cpu().numpy(), ei[:, up].astype(np.int32))
    assert np.array_equal(g.col.cpu().numpy(), ei[1].astype(np.int32))
    pairptr = np.concatenate([[0], np.cumsum(np.bincount(ei[0][up], minlength=n))])
    assert np.array_equal(g.pairptr.cpu().numpy(), pairptr)
    gc = _graph(pos, batch, r, False, 10 ** 6, with_pairs=True, capacity=g.num_edges + 64)
    E, P = g.num_edges, g.num_pairs
    assert int(gc.flags.item()) == 0
    assert torch.equal(gc.edge_index[:, :E], g.edge_index)
    assert torch.equal(gc.col[:E], g.col)
    assert torch.equal(gc.pair_ij[:, :P], g.pair_ij)
    assert torch.equal(gc.pairptr, g.pairptr)
    assert torch.equal(gc.eid2pair[:E], g.eid2pair)


@pytest.mark.parametrize("frac", [0.0, 0.37, 0.999])
def test_capacity_too_small(frac):
    """Edges past the capacity are dropped (flag 2); the ones written are the
    exact graph's first `capacity` edges and the CSR is clamped to them."""
    pos, batch, r = _case("long_rows")
    n = pos.shape[0]
    ref, _ = oracle_radius.radius_graph(pos, r, batch, False, 10 ** 6)
    cap = int(ref.shape[1] * frac)
    gc = _graph(pos, batch, r, False, 10 ** 6, capacity=cap)
    assert int(gc.flags.item()) & 2
    assert np.array_equal(gc.edge_index.cpu().numpy(), ref[:, :cap])
    assert np.array_equal(gc.rowptr.cpu().numpy(), np.minimum(_rowptr_ref(ref, n), cap))


@pytest.mark.parametrize("name,mnn", [("ragged", 1000), ("long_rows", 40)])
def test_exclusions_both_forms(name, mnn):
    from mlcg_amd import ops

    pos, batch, r = _case(name)
    n = pos.shape[0]
    rng = np.random.default_rng(5)
    m = 4 * n
    x = rng.integers(0, n, m)
    y = np.clip(x + rng.integers(-40, 41, m), 0, n - 1)
    exc = torch.from_numpy(np.stack([x, y]).astype(np.int64))
    xs, yptr = ops.exclusion_pair_to_ptr(exc, n)
    ref, _ = oracle_radius.radius_graph(pos, r, batch, False, mnn, exclude_pair_xs=xs.numpy(),
                                        ptr_exclude_pair_xs=yptr.numpy())
    kw = dict(exclude_pair_xs=xs.cuda(), ptr_exclude_pair_xs=yptr.cuda())
    g = _graph(pos, batch, r, False, mnn, **kw)
    assert np.array_equal(g.edge_index.cpu().numpy(), ref)
    gc = _graph(pos, batch, r, False, mnn, capacity=ref.shape[1] + 8, **kw)
    assert int(gc.flags.item()) & 2 == 0
    assert np.array_equal(gc.edge_index[:, :ref.shape[1]].cpu().numpy(), ref)
    assert np.array_equal(gc.rowptr.cpu().numpy(), _rowptr_ref(ref, n))


@pytest.mark.parametrize("name", ["long_rows", "ragged"])
def test_float64_both_forms(name):
    pos, batch, r = _case(name)
    pos = pos.astype(np.float64) * (1 + 1e-9)
    ref, _ = oracle_radius.radius_graph(pos, r, batch, True, 1000)
    g = _graph(pos, batch, r, True, 1000)
    assert np.array_equal(g.edge_index.cpu().numpy(), ref)
    gc = _graph(pos, batch, r, True, 1000, capacity=ref.shape[1] + 3)
    assert int(gc.flags.item()) == 0
    assert np.array_equal(gc.edge_index[:, :ref.shape[1]].cpu().numpy(), ref)


def test_empty_input():
    from mlcg_amd import ops

    for kw in ({}, {"capacity": 16}):
        g = ops.radius_graph(torch.zeros(0, 3, device="cuda"), 1.0,
                             batch=torch.zeros(0, dtype=torch.int64, device="cuda"),
                             max_num_neighbors=10, n_frames=0, **kw)
        assert g.rowptr.cpu().tolist() == [0] and int(g.flags.item()) == 0


def test_workspace_reused_across_sizes_and_forms():
    """One zero-filled workspace through a sequence of calls of both look-back
    entry points (mlcg_radius_rowptr, mlcg_radius_graph) whose row counts, and
    so block counts, rise, fall and rise again: every CSR and edge list equals
    the oracle's, the overflow word comes back cleared from garbage, and after
    each call the header counts the calls and the status words the next call
    will read are zero (no clearing launch between calls)."""
    from mlcg_amd import _lib, ops

    lib = _lib.load()
    seq = [("config3", "rowptr"), ("ragged", "graph"), ("long_rows", "rowptr"),
           ("config3", "graph"), ("mid_rows", "graph"), ("huge_frame", "rowptr"),
           ("config3", "rowptr")]
    cases = {name: _case(name) for name, _ in seq}
    n_max = max(c[0].shape[0] for c in cases.values())
    ws = torch.zeros(lib.mlcg_radius_workspace_bytes(n_max) // 8, dtype=torch.int64,
                     device="cuda")
    P = _lib.ptr
    for k, (name, form) in enumerate(seq):
        pos, batch, r = cases[name]
        n = pos.shape[0]
        print(f"call {k}: {name} n={n} {form}", flush=True)
        ref, _ = oracle_radius.radius_graph(pos, r, batch, False, 1000)
        E = ref.shape[1]
        p = torch.from_numpy(pos).cuda()
        b = torch.from_numpy(batch).cuda()
        fptr = ops.frame_ptr_from_batch(b, int(batch.max()) + 1)
        rowptr = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
        flags = torch.full((1,), 99, dtype=torch.int32, device="cuda")
        if form == "rowptr":
            st = lib.mlcg_radius_rowptr(P(p), P(b), P(fptr), n, r, 0, 1000, None, None,
                                        P(rowptr), None, P(ws), P(flags), _lib.stream_handle())
        else:
            cap = E + 16
            ei = torch.full((2, cap), -1, dtype=torch.int64, device="cuda")
            st = lib.mlcg_radius_graph(P(p), P(b), P(fptr), n, r, 0, 1000, None, None,
                                       P(rowptr), None, cap, cap, P(ei), None, 0, 0, None, None,
                                       P(ws), P(flags), _lib.stream_handle())
        assert st == 0
        torch.cuda.synchronize()
        assert int(flags.item()) == 0
        assert np.array_equal(rowptr.cpu().numpy(), _rowptr_ref(ref, n))
        if form == "graph":
            assert np.array_equal(ei[:, :E].cpu().numpy(), ref)
        epoch, mark = ws[:2].cpu().tolist()
        assert epoch == k + 1 and mark > 0
        nxt = ws[2 + ((k + 1) & 1)::2][:mark]
        assert int(nxt.abs().max().item()) == 0
