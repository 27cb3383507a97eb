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


# ---------------------------------------------------------------------------
# Pair exclusion (radius.cu:113-133 with the CSR of exclusion_pairs.cpp:7-62)

def _exclusions(rng, n, m, batch=None, symmetric=False):
    x = rng.integers(0, n, m)
    y = rng.integers(0, n, m)
    if batch is not None:  # mostly same-frame pairs, so that they bite
        y = np.where(rng.random(m) < 0.8, np.clip(x + rng.integers(-6, 7, m), 0, n - 1), y)
    exc = np.stack([x, y]).astype(np.int64)
    if symmetric:
        exc = np.concatenate([exc, exc[::-1]], axis=1)
    return exc


@pytest.mark.parametrize("n,split,loop,mnn", [(100, (100,), False, 100),
                                              (100, (10, 20, 100), True, 100),
                                              (300, (30, 60, 100), False, 5),
                                              (1, (100,), True, 10)])
def test_radius_exclusions_bit_exact(n, split, loop, mnn):
    from mlcg_amd import ops

    rng = np.random.default_rng(77 + n + mnn)
    pos = (4.0 * rng.random((n, 3))).astype(np.float32)
    batch = _batch(n, split)
    exc = _exclusions(rng, n, 4 * n, batch)
    exc = np.concatenate([exc, [[0, 0], [0, n + 3]]], axis=1)  # a self pair, a stray centre
    print(f"exclusions n={n} split={split} loop={loop} mnn={mnn}", flush=True)
    xs_ref, yp_ref = oracle_radius.exclusion_pair_to_ptr(exc, n)
    ref, _ = oracle_radius.radius_graph(pos, 2.0, batch, loop, mnn, exclude_pair_xs=xs_ref,
                                        ptr_exclude_pair_xs=yp_ref)
    xs, yp = ops.exclusion_pair_to_ptr(torch.from_numpy(exc).cuda(), n)
    assert xs.is_cuda and yp.is_cuda
    g = ops.radius_graph(torch.from_numpy(pos).cuda(), 2.0, batch=torch.from_numpy(batch).cuda(),
                         loop=loop, max_num_neighbors=mnn, exclude_pair_xs=xs,
                         ptr_exclude_pair_xs=yp)
    assert np.array_equal(g.edge_index.cpu().numpy(), ref)


def test_radius_cuda_mirror():
    """mlcg::radius_cuda's argument list (ptr_x frames, ignore_same_index,
    exclusion CSR): edges bit-exact against the oracle, distances within the
    reference test's 1e-6 (test_radius.py:66-104)."""
    from mlcg_amd.neighbor_list.radius import exclusion_pair_to_ptr, radius_cuda

    rng = np.random.default_rng(9)
    n = 200
    pos = (3.0 * rng.random((n, 3))).astype(np.float32)
    batch = _batch(n, (25, 50, 100))
    ptr_x = oracle_radius.frame_ptr_from_batch(batch)
    exc = _exclusions(rng, n, 500, batch)
    xs_ref, yp_ref = oracle_radius.exclusion_pair_to_ptr(exc, n)
    for ignore_same in (True, False):
        for use_excl in (False, True):
            kw = dict(exclude_pair_xs=xs_ref, ptr_exclude_pair_xs=yp_ref) if use_excl else {}
            ref, _ = oracle_radius.radius_graph(pos, 1.5, batch, not ignore_same, 32, **kw)
            xs, yp = (exclusion_pair_to_ptr(torch.from_numpy(exc).cuda(), n) if use_excl
                      else (None, None))
            x = torch.from_numpy(pos).cuda()
            ei, d = radius_cuda(x, torch.from_numpy(ptr_x).cuda(), 1.5, 32, ignore_same, xs, yp)
            assert np.array_equal(ei.cpu().numpy(), ref)
            want = np.linalg.norm(pos[ref[0]] - pos[ref[1]], axis=1)
            assert np.all(np.abs(d.cpu().numpy() - want) < 1e-6)


def test_radius_distance_exclusions_gradcheck():
    from torch.autograd import gradcheck, gradgradcheck

    from mlcg_amd.neighbor_list.radius import radius_distance

    torch.manual_seed(4)
    x = (2.0 * torch.rand(12, 3, dtype=torch.float64, device="cuda")).requires_grad_(True)
    exc = torch.tensor([[0, 1, 2, 5], [1, 0, 3, 4]], dtype=torch.int64, device="cuda")
    d, ei = radius_distance(x, 1.5, exclude_pair_indices=exc)
    pairs = set(zip(*ei.tolist()))
    assert not pairs & {(1, 0), (0, 1), (3, 2), (4, 5)}
    d_all, ei_all = radius_distance(x, 1.5)
    assert pairs == set(zip(*ei_all.tolist())) - {(1, 0), (0, 1), (3, 2), (4, 5)}
    f = lambda z: radius_distance(z, 1.5, exclude_pair_indices=exc)[0]
    assert gradcheck(f, (x,), eps=1e-7, atol=1e-6, nondet_tol=1e-7)
    assert gradgradcheck(f, (x,), eps=1e-7, atol=1e-6, nondet_tol=1e-7)


def test_pair_graph_with_symmetric_exclusions():
    """Bonded-neighbour exclusions (|i - j| <= 2 inside a chain, both
    directions): the pair structures stay consistent and the edges match
    the oracle."""
    from mlcg_amd import ops, synthetic

    b = synthetic.config2(n_frames=8)
    n = b.pos.shape[0]
    i = np.arange(n)
    same = lambda a, c: (c < n) & (b.batch[np.minimum(c, n - 1)] == b.batch[a])
    pairs = [np.stack([i[same(i, i + k)] + k, i[same(i, i + k)]]) for k in (1, 2)]
    exc = np.concatenate(pairs + [p[::-1] for p in pairs], axis=1).astype(np.int64)
    xs_ref, yp_ref = oracle_radius.exclusion_pair_to_ptr(exc, n)
    ref, _ = oracle_radius.radius_graph(b.pos, 20.0, b.batch, False, 1000,
                                        exclude_pair_xs=xs_ref, ptr_exclude_pair_xs=yp_ref)
    xs, yp = ops.exclusion_pair_to_ptr(torch.from_numpy(exc).cuda(), n)
    g = ops.radius_graph(torch.from_numpy(b.pos).cuda(), 20.0,
                         batch=torch.from_numpy(b.batch).cuda(), max_num_neighbors=1000,
                         with_pairs=True, exclude_pair_xs=xs, ptr_exclude_pair_xs=yp)
    ei = g.edge_index.cpu().numpy()
    assert np.array_equal(ei, ref)
    assert not np.any(np.abs(ei[0] - ei[1]) <= 2)
    pij = g.pair_ij.cpu().numpy()
    e2p = g.eid2pair.cpu().numpy()
    assert g.num_pairs * 2 == g.num_edges
    assert np.array_equal(np.minimum(ei[0], ei[1]), pij[0][e2p])
    assert np.array_equal(np.maximum(ei[0], ei[1]), pij[1][e2p])


def test_pair_graph_rejects_asymmetric_exclusions():
    from mlcg_amd import ops

    rng = np.random.default_rng(1)
    pos = torch.from_numpy((rng.random((20, 3))).astype(np.float32)).cuda()
    exc = torch.tensor([[3], [2]], dtype=torch.int64, device="cuda")  # drops (2, 3) only
    xs, yp = ops.exclusion_pair_to_ptr(exc, 20)
    g = ops.radius_graph(pos, 5.0, max_num_neighbors=100, exclude_pair_xs=xs,
                         ptr_exclude_pair_xs=yp)
    assert g.num_edges == 20 * 19 - 1
    with pytest.raises(RuntimeError, match="not symmetric"):
        ops.radius_graph(pos, 5.0, max_num_neighbors=100, with_pairs=True,
                         exclude_pair_xs=xs, ptr_exclude_pair_xs=yp)
    g = ops.radius_graph(pos, 5.0, max_num_neighbors=100, with_pairs=True, capacity=1024,
                         exclude_pair_xs=xs, ptr_exclude_pair_xs=yp)
    assert int(g.flags.item()) & 4


@pytest.mark.parametrize("method", ["torch", "custom_kernel", "hip"])
def test_atomic_data2neighbor_list_dict(method):
    """The reference's plugin point (neighbor_list.py:27-102): every backend
    name the switch accepts yields the NL dict of the reference -- tag,
    order 2, index_mapping [2, E] int64 equal to the oracle's edge list,
    cell_shifts zeros [E, 3], rcut, self_interaction, mapping_batch =
    batch[i] -- and SchNet accepts it as compatible; an unknown name raises."""
    from mlcg_amd import nn, synthetic
    from mlcg_amd.neighbor_list.neighbor_list import (atomic_data2neighbor_list,
                                                      hip_neighbor_list, validate_neighborlist)

    b = synthetic.config2(n_frames=6)
    data = b.to_torch("cuda")
    ei_ref, _ = oracle_radius.radius_graph(b.pos, 20.0, b.batch, False, 1000)
    nl = atomic_data2neighbor_list(data, 20.0, self_interaction=False, max_num_neighbors=1000,
                                   nls_distance_method=method)
    assert validate_neighborlist(nl)
    assert nl["order"] == 2 and nl["rcut"] == 20.0 and nl["self_interaction"] is False
    assert nl["tag"] == "nonbounded rc:20.0 order:2"
    assert nl["index_mapping"].dtype == torch.int64
    assert torch.equal(nl["index_mapping"].cpu(), torch.from_numpy(ei_ref))
    E = ei_ref.shape[1]
    assert tuple(nl["cell_shifts"].shape) == (E, 3) and not bool(nl["cell_shifts"].any())
    assert torch.equal(nl["mapping_batch"].cpu(), torch.from_numpy(b.batch[ei_ref[0]]))
    i, j, shifts, mask = hip_neighbor_list(data, 20.0)
    assert torch.equal(torch.stack([i, j]).cpu(), torch.from_numpy(ei_ref)) and bool(mask.all())
    rbf = nn.GaussianBasis(nn.CosineCutoff(0.0, 20.0), num_rbf=50)
    model = nn.StandardSchNet(rbf, nn.CosineCutoff(0.0, 20.0), [64], nls_distance_method=method)
    assert model.is_nl_compatible(nl)
    assert torch.equal(model.neighbor_list(data, 20.0)["SchNet"]["index_mapping"],
                       nl["index_mapping"])
    with pytest.raises(ValueError, match="not supported"):
        atomic_data2neighbor_list(data, 20.0, nls_distance_method="nvalchemi")


@pytest.mark.parametrize("n,x_range,r,split,loop", list(product(X, X_RANGE, R, BATCH_SIZES, LOOP)))
def test_radius_f64_sweep_bit_exact(n, x_range, r, split, loop):
    """float64 positions (the reference's own test sweep runs its kernel in
    float64, test_radius.py:66-104): the HIP double search equals the C
    oracle's double search bit for bit."""
    rng = np.random.default_rng(3000 + n)
    lo, hi = x_range
    pos = (hi - lo) * rng.random((n, 3)) + lo
    batch = _batch(n, split)
    ei_ref, _ = oracle_radius.radius_graph(pos, r, batch, loop, 1000)
    g = _hip(pos, r, batch, loop, 1000)
    assert np.array_equal(g.edge_index.cpu().numpy(), ei_ref)


def test_radius_cuda_float64_boundary():
    """radius_cuda on float64 positions decides membership in double: a pair
    one double ulp inside the cutoff is kept, although float32 rounding would
    put it on the cutoff; the distances come back in float64."""
    from mlcg_amd.neighbor_list.radius import radius_cuda

    x = float(np.nextafter(1.0, 0.0))
    pos = torch.tensor([[0.0, 0, 0], [x, 0, 0], [0.0, 0, 0], [1.0, 0, 0]],
                       dtype=torch.float64, device="cuda")
    ptr = torch.tensor([0, 2, 4], device="cuda")
    ei, d = radius_cuda(pos, ptr, 1.0, 8, True)
    assert ei.cpu().tolist() == [[0, 1], [1, 0]] and d.dtype == torch.float64
    ei32, _ = radius_cuda(pos.float(), ptr, 1.0, 8, True)
    assert ei32.shape[1] == 0
    with pytest.raises(RuntimeError, match="float32, float64, float16 or bfloat16"):
        radius_cuda(pos.to(torch.int32), ptr, 1.0, 8, True)


def _narrow(dt):
    return torch.float16 if dt == "f16" else torch.bfloat16


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("loop,mnn,excl", [(False, 1000, False), (True, 1000, False),
                                           (False, 6, False), (False, 1000, True)])
def test_radius_narrow_positions_bit_exact(dt, loop, mnn, excl):
    """float16 / bfloat16 positions (the reference's Half / BFloat16 dispatch,
    radius.cu:243-250): the HIP search, every operation rounded to the 16-bit
    type, equals the C oracle's bit for bit on 16 globule frames of 100 beads,
    with self loops, a binding max_num_neighbors and exclusions; and the
    16-bit membership differs from the float32 search of the same (widened)
    positions, so the comparison is sensitive to the arithmetic."""
    from mlcg_amd import ops, synthetic

    rng = np.random.default_rng(500 + mnn + 7 * loop + 3 * excl)
    pos32 = synthetic.globule(16, 100, 12.0, rng).reshape(-1, 3).astype(np.float32)
    x = torch.from_numpy(pos32).to(_narrow(dt))
    bits = x.view(torch.int16).numpy().view(np.uint16)
    n = x.shape[0]
    batch = np.repeat(np.arange(16), 100)
    r = 9.7
    kw_ref, kw = {}, {}
    if excl:
        exc = _exclusions(rng, n, 4 * n, batch)
        xs_ref, yp_ref = oracle_radius.exclusion_pair_to_ptr(exc, n)
        kw_ref = dict(exclude_pair_xs=xs_ref, ptr_exclude_pair_xs=yp_ref)
        xs, yp = ops.exclusion_pair_to_ptr(torch.from_numpy(exc).cuda(), n)
        kw = dict(exclude_pair_xs=xs, ptr_exclude_pair_xs=yp)
    print(f"narrow {dt} loop={loop} mnn={mnn} excl={excl}", flush=True)
    ref, _ = oracle_radius.radius_graph_narrow(bits, dt, r, batch, loop, mnn, **kw_ref)
    g = ops.radius_graph(x.cuda(), r, batch=torch.from_numpy(batch).cuda(), loop=loop,
                         max_num_neighbors=mnn, n_frames=16, **kw)
    assert np.array_equal(g.edge_index.cpu().numpy(), ref)
    if mnn == 1000 and not excl and not loop:
        wide, _ = oracle_radius.radius_graph(x.float().numpy(), r, batch, loop, mnn)
        assert not np.array_equal(wide, ref)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_radius_cuda_narrow_distances(dt):
    """mlcg::radius_cuda on 16-bit positions: the oracle's edge list, and the
    distances in x's type as the reference's kernel forms them (each
    operation rounded to the 16-bit type, then sqrt), equal to a float32
    computation rounded once within one 16-bit ulp."""
    from mlcg_amd import library, synthetic

    library.register()
    rng = np.random.default_rng(77)
    pos32 = synthetic.globule(4, 60, 9.0, rng).reshape(-1, 3).astype(np.float32)
    x = torch.from_numpy(pos32).to(_narrow(dt)).cuda()
    ptr = torch.tensor([0, 60, 120, 180, 240], device="cuda")
    ei, d = torch.ops.mlcg.radius_cuda(x, ptr, 7.5, 64, True)
    bits = x.cpu().view(torch.int16).numpy().view(np.uint16)
    ref, _ = oracle_radius.radius_graph_narrow(bits, dt, 7.5, np.repeat(np.arange(4), 60),
                                               False, 64)
    assert np.array_equal(ei.cpu().numpy(), ref) and d.dtype == x.dtype
    xc = x.cpu()
    diff = xc[ei[1].cpu()] - xc[ei[0].cpu()]
    sq = diff * diff
    want = torch.sqrt((sq[:, 0] + sq[:, 1]) + sq[:, 2])
    assert torch.equal(d.cpu(), want)
    once = (xc.float()[ei[1].cpu()] - xc.float()[ei[0].cpu()]).norm(dim=1)
    ulp = 2.0 ** -10 if dt == "f16" else 2.0 ** -7
    assert float(((d.cpu().float() - once).abs() / once).max()) < 4 * ulp


def test_registered_operators_and_torch_compile():
    """torch.ops.mlcg.radius_cuda and exclusion_pair_to_ptr (the reference's
    registered operator names, radius.cu:313-314, exclusion_pairs.cpp:64-65)
    give the wrappers' results, also inside torch.compile(fullgraph=True) --
    traced through the fake kernels -- as the reference's simulation compiles
    its model (simulation/base.py:447-490)."""
    import mlcg_amd  # noqa: F401
    from mlcg_amd import ops
    from mlcg_amd.neighbor_list.radius import radius_cuda

    rng = np.random.default_rng(5)
    pos = torch.from_numpy(rng.random((300, 3)) * 8.0).float().cuda()
    ptr = torch.tensor([0, 100, 300], device="cuda")
    ei, d = torch.ops.mlcg.radius_cuda(pos, ptr, 2.5, 64, True)
    ei2, d2 = radius_cuda(pos, ptr, 2.5, 64, True)
    assert torch.equal(ei, ei2) and torch.equal(d, d2)
    exc = torch.tensor([[1, 2, 2, 5], [0, 0, 3, 4]], device="cuda")
    xs, p = torch.ops.mlcg.exclusion_pair_to_ptr(exc, 6)
    xs2, p2 = ops.exclusion_pair_to_ptr(exc, 6)
    assert torch.equal(xs, xs2) and torch.equal(p, p2)

    def per_frame_sum(x, ptr_x):
        e, dist = torch.ops.mlcg.radius_cuda(x, ptr_x, 2.5, 64, True)
        frame = torch.searchsorted(ptr_x, e[0], right=True) - 1
        return torch.zeros(2, device=x.device, dtype=x.dtype).index_add(0, frame, dist)

    torch._dynamo.reset()
    compiled = torch.compile(per_frame_sum, backend="aot_eager", fullgraph=True)
    assert torch.allclose(compiled(pos, ptr), per_frame_sum(pos, ptr), rtol=1e-6, atol=0)


def test_compiled_schnet_matches_eager():
    """torch.compile of the module (the reference's simulation path,
    simulation/base.py:447-490; its differential test is eager against
    compiled, tests/unit/simulation/test_compilation.py:229-270, rtol = atol =
    1e-5): the fused HIP forward and forces run under the compiler (which
    treats the kernel launches as opaque calls) and give the eager energies
    and forces."""
    from mlcg_amd import nn, synthetic

    torch.manual_seed(3)
    rbf = nn.GaussianBasis(nn.CosineCutoff(0.0, 20.0), num_rbf=50)
    model = nn.GradientsOut(nn.StandardSchNet(rbf, nn.CosineCutoff(0.0, 20.0), [64])).cuda()
    model.eval()
    data = synthetic.config2(n_frames=8).to_torch("cuda")
    ref = model(data.clone())
    E0, F0 = ref.out["SchNet"]["energy"].clone(), ref.out["SchNet"]["forces"].clone()
    torch._dynamo.reset()
    compiled = torch.compile(model, backend="aot_eager")
    out = compiled(data.clone())
    assert torch.allclose(out.out["SchNet"]["energy"], E0, rtol=1e-5, atol=1e-5)
    assert torch.allclose(out.out["SchNet"]["forces"], F0, rtol=1e-5, atol=1e-5)
