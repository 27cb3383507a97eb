"""Fused HIP SchNet against the CPU oracle (oracle/schnet_ref.py).

Tolerances, per element (tests.helpers.check:
|got - ref| <= rtol |ref| + rtol / 10 * max|ref|):
  energies / forces   rtol 1e-5 (absolute term 1e-6 of the largest element)
  force-matching grads rtol 1e-4 (absolute term 1e-5 of the tensor's largest)
The oracle runs in fp64 (the mathematically exact target); the HIP path is
fp32.  Where the reference's own fp32 arithmetic differs from fp64 by more
than the tolerance (never at these sizes), the test says so.
"""

import numpy as np
import pytest
import torch

from oracle import radius as oracle_radius
from oracle import schnet_ref as R
from tests.helpers import (check, check_calibrated, close_report, make_cfg, make_model, max_abs,
                           rel_err, scaled_atol)

pytestmark = pytest.mark.gpu


def _small_batch(n_frames=6, n_beads=14, seed=3):
    from mlcg_amd import synthetic

    rng = np.random.default_rng(seed)
    pos = synthetic.self_avoiding_walk(n_frames, n_beads, rng)
    types = rng.integers(1, 21, size=(n_frames, n_beads))
    forces = rng.standard_normal((n_frames * n_beads, 3)).astype(np.float32)
    return synthetic._flatten(pos, types, seed, forces)


def _oracle_inputs(b, rc, dtype=torch.float64):
    ei, _ = oracle_radius.radius_graph(b.pos, rc, b.batch, False, 1000)
    return (torch.from_numpy(b.pos).to(dtype), torch.from_numpy(b.atom_types),
            torch.from_numpy(b.batch), torch.from_numpy(ei))


@pytest.mark.parametrize("num_rbf", [10, 50, 64, 65, 100])
def test_filter_kernel_matches_torch(num_rbf):
    """The filter forward (K <= 64: products on the fp16 MFMA with split
    operands; wider bases: fp32 MFMA) against fp64 torch, every element
    within 1e-5 of the tensor's largest (W' = dW/dd sums cancelling terms:
    torch's own fp32 arithmetic errs by 8.6e-7 of max|W'| at config 2)."""
    from mlcg_amd import ops, synthetic

    cfg = make_cfg(num_blocks=1, rc=20.0, num_rbf=num_rbf)
    sd = R.random_state_dict(cfg, seed=11)
    b = synthetic.config2(n_frames=8)
    pos = torch.from_numpy(b.pos).cuda()
    g = ops.radius_graph(pos, 20.0, torch.from_numpy(b.batch).cuda(), max_num_neighbors=1000,
                         with_pairs=True)
    model = make_model(cfg, sd)
    spec = model.fused_spec()
    blk = model.fused_params().blocks[0]
    W, Wd, dist = ops.filter_fwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2)
    Ws, Wds, _ = ops.filter_fwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2, strict_fp32=True)
    # fp64 torch reference on the same pairs
    pij = g.pair_ij.long().cpu()
    p64 = torch.from_numpy(b.pos).double()
    d = (p64[pij[1]] - p64[pij[0]]).norm(dim=1).requires_grad_(True)
    sd64 = R.to_dtype(sd, torch.float64)
    rbf = R.gaussian_rbf(d, sd64["rbf_layer.offset"], sd64["rbf_layer.coeff"],
                         R.Cutoff("cosine", 0.0, 20.0))
    layers = R._layers(sd64, "interaction_blocks.0.conv.filter_network")
    Wr = R.mlp(rbf, layers, torch.tanh) * R.cosine_cutoff(d, 0.0, 20.0).view(-1, 1)
    Wdr = torch.stack([torch.autograd.grad(Wr[:, f].sum(), d, retain_graph=True)[0]
                       for f in range(128)], dim=1)
    print("W rel", rel_err(W, Wr), "Wd rel", rel_err(Wd, Wdr),
          "dist", max_abs(dist, d.detach()))
    print("strict fp32: W rel", rel_err(Ws, Wr), "Wd rel", rel_err(Wds, Wdr))
    check(W, Wr.detach(), 1e-5, 'W', atol_frac=1.0)
    check(Wd, Wdr, 1e-5, 'Wd', atol_frac=1.0)
    check(Ws, Wr.detach(), 1e-5, 'Ws', atol_frac=1.0)
    check(Wds, Wdr, 1e-5, 'Wds', atol_frac=1.0)
    assert max_abs(dist, d.detach()) < 1e-5


def test_gather_matches_index_add():
    from mlcg_amd import ops, synthetic

    b = synthetic.config2(n_frames=8)
    pos = torch.from_numpy(b.pos).cuda()
    g = ops.radius_graph(pos, 20.0, torch.from_numpy(b.batch).cuda(), max_num_neighbors=1000,
                         with_pairs=True)
    torch.manual_seed(0)
    y = torch.randn(pos.shape[0], 128, device="cuda")
    W = torch.randn(g.num_pairs, 128, device="cuda")
    out = ops.cfconv_gather(y, W, g)
    ei = g.edge_index
    We = W[g.eid2pair.long()].double()
    # float64 reference (exact to ~1e-16 whatever index_add's order); the fp32
    # sum of a row's n terms, in any order, lies within gamma_n sum |terms|
    # of it (recursive summation, gamma_n = n u / (1 - n u), u = 2^-24, the
    # products' own rounding counted as one more term)
    terms = y[ei[0]].double() * We
    ref = torch.zeros_like(y, dtype=torch.float64).index_add_(0, ei[1], terms)
    mag = torch.zeros_like(ref).index_add_(0, ei[1], terms.abs())
    n = int(torch.diff(g.rowptr.long()).max().item()) + 1
    u = 2.0 ** -24
    bound = (n * u / (1 - n * u)) * mag
    err = (out.double() - ref).abs()
    worst = float((err / bound.clamp_min(1e-300)).max())
    print(f"gather: worst error / summation bound = {worst:.3g} (rows up to {n - 1} edges)")
    assert bool((err <= bound).all()), worst


@pytest.mark.parametrize("act", ["tanh", "ssp"])
def test_energy_forces_small(act):
    from mlcg_amd import nn

    cfg = make_cfg(num_blocks=3, rc=12.0, act=act)
    sd = R.random_state_dict(cfg, seed=5)
    b = _small_batch()
    pos64, types, batch, ei = _oracle_inputs(b, 12.0)
    E_ref, F_ref = R.schnet_energy_forces(R.to_dtype(sd, torch.float64), cfg, pos64, types,
                                          batch, ei, b.n_frames)
    E32, F32 = R.schnet_energy_forces(sd, cfg, pos64.float(), types, batch, ei, b.n_frames)
    model = make_model(cfg, sd)
    gm = nn.GradientsOut(model).eval()
    data = b.to_torch("cuda")
    data = gm(data)
    E = data.out["SchNet"]["energy"]
    F = data.out["SchNet"]["forces"]
    check_calibrated(E, E_ref, E32, 1e-5, 'E')
    check_calibrated(F, F_ref, F32, 1e-5, 'F')
    assert torch.allclose(E.double().cpu(), E_ref, rtol=1e-5, atol=1e-6 * float(E_ref.abs().max()))


def test_energy_plain_forward_and_autograd_forces():
    """SchNet.forward + torch.autograd.grad (generic GradientsOut path)."""
    cfg = make_cfg(num_blocks=2, rc=12.0)
    sd = R.random_state_dict(cfg, seed=9)
    b = _small_batch()
    pos64, types, batch, ei = _oracle_inputs(b, 12.0)
    E_ref, F_ref = R.schnet_energy_forces(R.to_dtype(sd, torch.float64), cfg, pos64, types,
                                          batch, ei, b.n_frames)
    model = make_model(cfg, sd)
    data = b.to_torch("cuda")
    data.pos.requires_grad_(True)
    data = model(data)
    E = data.out["SchNet"]["energy"]
    (g,) = torch.autograd.grad(E.sum(), data.pos)
    check(E, E_ref, 1e-5, 'E')
    check(-g, F_ref, 1e-5, '-g')


def _param_grads(model):
    return {k: p.grad for k, p in model.named_parameters()}


@pytest.mark.parametrize("act", ["tanh", "ssp"])
def test_force_matching_grads_small(act):
    from mlcg_amd import nn

    cfg = make_cfg(num_blocks=3, rc=12.0, act=act)
    sd = R.random_state_dict(cfg, seed=13)
    b = _small_batch()
    pos64, types, batch, ei = _oracle_inputs(b, 12.0)
    fref64 = torch.from_numpy(b.forces).double()
    loss_ref, _, _, g_ref = R.force_matching_grads(R.to_dtype(sd, torch.float64), cfg, pos64,
                                                   types, batch, ei, b.n_frames, fref64)
    model = make_model(cfg, sd)
    gm = nn.GradientsOut(model).train()
    data = b.to_torch("cuda")
    data = gm(data)
    loss = torch.nn.functional.mse_loss(data.out["SchNet"]["forces"], data.forces)
    loss.backward()
    assert abs(float(loss) - float(loss_ref)) <= 1e-5 * abs(float(loss_ref))
    grads = _param_grads(model)
    worst = 0.0
    for k, gr in g_ref.items():
        got = grads[k]
        assert got is not None, k
        worst = max(worst, check(got, gr, 1e-4, k))
    print(act, "worst param-grad ratio", worst)


def test_generic_double_backward():
    """autograd.grad(E, pos, create_graph=True) then a force loss backward
    through the fused Energy/EnergyGrad functions."""
    cfg = make_cfg(num_blocks=2, rc=12.0)
    sd = R.random_state_dict(cfg, seed=17)
    b = _small_batch()
    pos64, types, batch, ei = _oracle_inputs(b, 12.0)
    fref64 = torch.from_numpy(b.forces).double()
    _, _, _, g_ref = R.force_matching_grads(R.to_dtype(sd, torch.float64), cfg, pos64, types,
                                            batch, ei, b.n_frames, fref64)
    model = make_model(cfg, sd)
    data = b.to_torch("cuda")
    data.pos.requires_grad_(True)
    data = model(data)
    E = data.out["SchNet"]["energy"]
    (g,) = torch.autograd.grad(E.sum(), data.pos, create_graph=True)
    loss = torch.nn.functional.mse_loss(-g, data.forces)
    loss.backward()
    grads = _param_grads(model)
    for k, gr in g_ref.items():
        check(grads[k], gr, 1e-4, k)


def test_config1_cpu_reference_case():
    """Config 1 (1 block, SSP, 30 A) energies and forces."""
    from mlcg_amd import nn, synthetic

    cfg = make_cfg(num_blocks=1, rc=30.0, act="ssp")
    sd = R.random_state_dict(cfg, seed=synthetic.seed_for(1))
    b = synthetic.config1()
    pos64, types, batch, ei = _oracle_inputs(b, 30.0)
    E_ref, F_ref = R.schnet_energy_forces(R.to_dtype(sd, torch.float64), cfg, pos64, types,
                                          batch, ei, b.n_frames)
    E32, F32 = R.schnet_energy_forces(sd, cfg, pos64.float(), types, batch, ei, b.n_frames)
    model = make_model(cfg, sd)
    data = nn.GradientsOut(model).eval()(b.to_torch("cuda"))
    check(data.out["SchNet"]["energy"], E_ref, 1e-5, 'data.out["SchNet"]["energy"]')
    check(data.out["SchNet"]["forces"], F_ref, 1e-5, 'data.out["SchNet"]["forces"]')
    # the literal reading of the bar (absolute term 1e-6 rather than 1e-6 of
    # the largest element), for the kernels and for the reference's own fp32
    for name, got, r32, r in (("energy", data.out["SchNet"]["energy"], E32, E_ref),
                              ("forces", data.out["SchNet"]["forces"], F32, F_ref)):
        n_hip, n, _, _ = close_report(got, r, 1e-5, 1e-6)
        n_ref, _, _, _ = close_report(r32, r, 1e-5, 1e-6)
        print(f"config 1 {name}: {n_hip}/{n} elements outside rtol 1e-5 + literal atol 1e-6 "
              f"(the reference's fp32 arithmetic: {n_ref}/{n})")


def test_golden_fixture_hip():
    """HIP path against the committed fp64 oracle fixture (hidden 16, 16 RBF,
    2 blocks; tests/golden/make_golden.py): energies, forces and every
    force-matching parameter gradient.  The energies (0.25, -0.017, 0.42) are
    sums of cancelling per-node terms: the reference's own fp32 arithmetic
    errs by 5.4e-7 = 1.3e-6 of max|E| on them, so each energy is held to 1e-5
    of the largest (atol_frac=1.0)."""
    import os

    from mlcg_amd import nn

    g = torch.load(os.path.join(os.path.dirname(__file__), "golden", "schnet_small.pt"),
                   weights_only=True)
    cfg = R.SchNetConfig(**g["cfg"])
    sd = {k: v.float() for k, v in g["state_dict"].items()}
    rbf = nn.GaussianBasis(nn.CosineCutoff(0.0, cfg.rbf_hi), num_rbf=cfg.num_rbf)
    model = nn.StandardSchNet(rbf, nn.CosineCutoff(0.0, cfg.conv_hi), [8], hidden_channels=16,
                              embedding_size=sd["embedding_layer.weight"].shape[0],
                              num_filters=128, num_interactions=cfg.num_blocks,
                              activation=torch.nn.Tanh())
    model.load_state_dict(sd)
    model = model.cuda()
    from mlcg_amd.data import AtomicData

    n_frames = int(g["n_frames"])
    data = AtomicData(pos=g["pos"].float().cuda(), atom_types=g["types"].cuda(),
                      batch=g["batch"].cuda(),
                      n_atoms=torch.bincount(g["batch"], minlength=n_frames).cuda(),
                      forces=g["forces_ref"].float().cuda())
    gm = nn.GradientsOut(model).train()
    data = gm(data)
    E, F = data.out["SchNet"]["energy"], data.out["SchNet"]["forces"]
    check(E, g["energy"], 1e-5, 'E', atol_frac=1.0)
    check(F, g["forces"], 1e-5, 'F')
    loss = torch.nn.functional.mse_loss(F, data.forces)
    loss.backward()
    assert abs(float(loss) - float(g["loss"])) <= 1e-5 * abs(float(g["loss"]))
    for k, p in model.named_parameters():
        check(p.grad, g["grads"][k], 1e-4, k)


def _config4_model(sd=None, seed=4):
    from mlcg_amd import nn

    cfg = make_cfg(num_blocks=3, rc=15.0)
    if sd is None:
        sd = R.random_state_dict(cfg, seed=seed)
    return cfg, sd, make_model(cfg, sd)


def test_fp16_filters_config4_vs_oracle():
    """Config 4 (globular 500-bead frames, rc 15 A, fp16 filter linears with
    fp32 accumulation): energies and forces within 2e-3 of the fp64 oracle on
    16 frames, per element relative to the tensor's largest element (fp16
    operands carry 11 significant bits, so a force component's error scales
    with the pair terms it sums), and norm-wise; the per-element count against
    a tighter absolute term is printed."""
    from mlcg_amd import nn, synthetic

    b = synthetic.config4(n_frames=16)
    cfg, sd, model = _config4_model()
    pos64, types, batch, ei = _oracle_inputs(b, 15.0)
    E_ref, F_ref = R.schnet_energy_forces(R.to_dtype(sd, torch.float64), cfg, pos64, types,
                                          batch, ei, b.n_frames)
    model.fp16_filters = True
    data = nn.GradientsOut(model).eval()(b.to_torch("cuda"))
    print("fp16 config4: edges", ei.shape[1])
    E16, F16 = data.out["SchNet"]["energy"], data.out["SchNet"]["forces"]
    check(E16, E_ref, 2e-3, "fp16 energy", atol_frac=1.0)
    check(F16, F_ref, 2e-3, "fp16 forces", atol_frac=1.0)
    # other readings of "2e-3 relative": norm-wise, and per element with the
    # absolute term a tenth of the bound's (2e-4 of the largest component)
    print(f"fp16 config4: norm-wise relative error: forces {rel_err(F16, F_ref):.3e}, "
          f"energies {rel_err(E16, E_ref):.3e}")
    n_el, n, _, _ = close_report(F16, F_ref, 2e-3, scaled_atol(F_ref, 2e-4))
    print(f"fp16 config4 forces: {n_el}/{n} components outside 2e-3 |ref| + 2e-4 max|ref|")
    assert rel_err(F16, F_ref) < 2e-3
    # and the fp32 path on the same frames meets the fp32 tolerance
    model.fp16_filters = False
    d32 = nn.GradientsOut(model).eval()(b.to_torch("cuda"))
    check(d32.out["SchNet"]["forces"], F_ref, 1e-5, 'd32.out["SchNet"]["forces"]')


def test_fp16_filters_config4_full_size_vs_fp32():
    """Full config 4 (256 x 500 beads, ~6M edges): fp16-filter forces within
    2e-3 of the fp32 HIP path (the fp32 path is pinned to the oracle above)."""
    from mlcg_amd import nn, synthetic

    b = synthetic.config4()
    _, _, model = _config4_model()
    data = b.to_torch("cuda")
    gm = nn.GradientsOut(model).eval()
    F32 = gm(data).out["SchNet"]["forces"].clone()
    model.fp16_filters = True
    F16 = gm(data).out["SchNet"]["forces"]
    print("fp16 vs fp32 forces at full config 4: edges", model.last_graph.num_edges)
    check(F16, F32, 2e-3, "fp16 forces vs fp32", atol_frac=1.0)
    print(f"fp16 vs fp32 at full config 4: norm-wise relative error {rel_err(F16, F32):.3e}")
    assert rel_err(F16, F32) < 2e-3


def _filter_setup(n_frames=8, seed=11, num_rbf=50):
    from mlcg_amd import ops, synthetic

    cfg = make_cfg(num_blocks=1, rc=20.0, num_rbf=num_rbf)
    sd = R.random_state_dict(cfg, seed=seed)
    b = synthetic.config2(n_frames=n_frames)
    pos = torch.from_numpy(b.pos).cuda()
    g = ops.radius_graph(pos, 20.0, torch.from_numpy(b.batch).cuda(), max_num_neighbors=1000,
                         with_pairs=True)
    model = make_model(cfg, sd)
    return cfg, sd, b, pos, g, model.fused_spec(), model.fused_params().blocks[0]


@pytest.mark.parametrize("num_rbf", [10, 50, 64, 65, 100])
def test_filter_bwd_matches_autograd(num_rbf):
    """Parameter gradients of <Wbar, W> + <Wdbar, dW/dd> from the fused
    backward kernel against fp64 autograd of the restated filter chain
    (K <= 64 and the wide K <= 128 kernel variant)."""
    from mlcg_amd import ops

    cfg, sd, b, pos, g, spec, blk = _filter_setup(num_rbf=num_rbf)
    P = g.num_pairs
    gen = torch.Generator(device="cuda").manual_seed(3)
    Wbar = torch.randn(P, 128, device="cuda", generator=gen)
    Wdbar = torch.randn(P, 128, device="cuda", generator=gen)
    dW1, db1, dW2 = ops.filter_bwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2, Wbar, Wdbar)
    gW1, gb1, gW2 = _filter_bwd_ref(sd, b, g, Wbar, Wdbar)
    print("dW1", rel_err(dW1, gW1), "db1", rel_err(db1, gb1), "dW2", rel_err(dW2, gW2))
    check(dW1, gW1, 1e-4, 'dW1')
    check(db1, gb1, 1e-4, 'db1')
    check(dW2, gW2, 1e-4, 'dW2')


def _filter_bwd_ref(sd, b, g, Wbar, Wdbar):
    """fp64 autograd of <Wbar, W> + <Wdbar, dW/dd> through the restated
    filter chain (Gaussian basis, tanh, cosine cutoffs at 20)."""
    pij = g.pair_ij.long().cpu()
    p64 = torch.from_numpy(b.pos).double()
    d = (p64[pij[1]] - p64[pij[0]]).norm(dim=1).requires_grad_(True)
    sd64 = R.to_dtype(sd, torch.float64)
    lay = R._layers(sd64, "interaction_blocks.0.conv.filter_network")
    for L_ in lay:
        for t in L_.values():
            t.requires_grad_(True)
    rbf = R.gaussian_rbf(d, sd64["rbf_layer.offset"], sd64["rbf_layer.coeff"],
                         R.Cutoff("cosine", 0.0, 20.0))
    Wr = R.mlp(rbf, lay, torch.tanh) * R.cosine_cutoff(d, 0.0, 20.0).view(-1, 1)
    # dW/dd contracted with Wdbar: d/dd of <Wdbar, W> per pair
    wd_term, = torch.autograd.grad((Wr * Wdbar.double().cpu()).sum(), d, create_graph=True)
    obj = (Wr * Wbar.double().cpu()).sum() + wd_term.sum()
    return torch.autograd.grad(obj, [lay[0]["weight"], lay[0]["bias"], lay[1]["weight"]])


def test_filter_bwd_adjoint_dynamic_range():
    """Adjoints whose size grows by 10^6 along the pair list, after a run of
    all-zero tiles: every workgroup meets a larger maximum on most of its
    tiles, so the split-operand pair reductions rescale their accumulators
    many times; the gradients still match fp64 autograd."""
    from mlcg_amd import ops

    cfg, sd, b, pos, g, spec, blk = _filter_setup(n_frames=64, seed=13)
    P = g.num_pairs
    gen = torch.Generator(device="cuda").manual_seed(4)
    ramp = torch.pow(10.0, torch.linspace(-4.0, 2.0, P, device="cuda"))
    ramp[: 16 * 300] = 0.0
    Wbar = torch.randn(P, 128, device="cuda", generator=gen) * ramp[:, None]
    Wdbar = torch.randn(P, 128, device="cuda", generator=gen) * ramp[:, None]
    dW1, db1, dW2 = ops.filter_bwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2, Wbar, Wdbar)
    gW1, gb1, gW2 = _filter_bwd_ref(sd, b, g, Wbar, Wdbar)
    print("P", P, "dW1", rel_err(dW1, gW1), "db1", rel_err(db1, gb1), "dW2", rel_err(dW2, gW2))
    check(dW1, gW1, 1e-4, 'dW1')
    check(db1, gb1, 1e-4, 'db1')
    check(dW2, gW2, 1e-4, 'dW2')


@pytest.mark.parametrize("num_rbf", [10, 50, 64, 65, 100])
def test_filter_bwd_cfconv_matches_explicit(num_rbf):
    """The node-adjoint backward equals the explicit one with the adjoints
    formed in torch."""
    from mlcg_amd import ops

    cfg, sd, b, pos, g, spec, blk = _filter_setup(n_frames=16, seed=12, num_rbf=num_rbf)
    N = pos.shape[0]
    gen = torch.Generator(device="cuda").manual_seed(5)
    g2, y, g1, yd = (torch.randn(N, 128, device="cuda", generator=gen) for _ in range(4))
    dd = torch.randn(g.pair_capacity, device="cuda", generator=gen)
    i, j = g.pair_ij.long()
    Wbar = g2[i] * y[j] + g2[j] * y[i] + g1[i] * yd[j] + g1[j] * yd[i]
    Wdbar = dd[:, None] * (g1[i] * y[j] + g1[j] * y[i])
    ref = ops.filter_bwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2, Wbar, Wdbar)
    got = ops.filter_bwd_cfconv(pos, g, spec.filt, blk.W1, blk.b1, blk.W2, g2, y, g1, yd, dd)
    for a, r in zip(got, ref):
        check(a, r, 1e-5, 'a')
    # without the tangent stream
    Wbar0 = g2[i] * y[j] + g2[j] * y[i]
    ref0 = ops.filter_bwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2, Wbar0,
                          torch.zeros_like(Wbar0))
    got0 = ops.filter_bwd_cfconv(pos, g, spec.filt, blk.W1, blk.b1, blk.W2, g2, y, None, None,
                                 None)
    for a, r in zip(got0, ref0):
        check(a, r, 1e-5, 'a')
    # tangent stream without ydot (the first block, whose input has no tangent)
    ref1 = ops.filter_bwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2, Wbar0, Wdbar)
    got1 = ops.filter_bwd_cfconv(pos, g, spec.filt, blk.W1, blk.b1, blk.W2, g2, y, g1, None,
                                 dd)
    for a, r in zip(got1, ref1):
        check(a, r, 1e-5, 'a')


def test_cosine_cutoff_with_lower_bound():
    """The CFConv envelope with cutoff_lower > 0 (cutoff.py:145-150:
    0.5 (cos(pi (2 (d - lo) / (hi - lo) + 1)) + 1) on lo < d < hi, zero
    elsewhere), with lo = 5 A so that the bonded pairs (3.8 A) fall below it:
    energies, forces and force-matching gradients against the fp64 oracle."""
    import warnings

    from mlcg_amd import nn

    cfg = make_cfg(num_blocks=2, rc=12.0, conv_lo=5.0)
    sd = R.random_state_dict(cfg, seed=23)
    b = _small_batch(seed=8)
    pos64, types, batch, ei = _oracle_inputs(b, 12.0)
    d = (pos64[ei[1]] - pos64[ei[0]]).norm(dim=1)
    assert int((d < 5.0).sum()) > 0 and int((d > 5.0).sum()) > 0
    fref64 = torch.from_numpy(b.forces).double()
    sd64 = R.to_dtype(sd, torch.float64)
    E_ref, F_ref = R.schnet_energy_forces(sd64, cfg, pos64, types, batch, ei, b.n_frames)
    loss_ref, _, _, g_ref = R.force_matching_grads(sd64, cfg, pos64, types, batch, ei,
                                                   b.n_frames, fref64)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")  # lower cutoffs of RBF and CFConv differ on purpose
        model = make_model(cfg, sd)
    assert model.fused_spec() is not None and model.fused_spec().filt.conv_lo == 5.0
    data = nn.GradientsOut(model).train()(b.to_torch("cuda"))
    E, F = data.out["SchNet"]["energy"], data.out["SchNet"]["forces"]
    check(E, E_ref, 1e-5, "energy (cosine lo 5)")
    check(F, F_ref, 1e-5, "forces (cosine lo 5)")
    loss = torch.nn.functional.mse_loss(F, data.forces)
    loss.backward()
    assert abs(float(loss) - float(loss_ref)) <= 1e-5 * abs(float(loss_ref))
    for k, gr in g_ref.items():
        check(dict(model.named_parameters())[k].grad, gr, 1e-4, k)


def test_mean_aggregation_vs_oracle():
    """CFConv with aggr="mean" (PyG's mean: the HIP gather divided by each
    receiver's in-degree, module by module) against the fp64 oracle's mean
    aggregation: energies and forces at 1e-5, and the force-matching
    parameter gradients (double backward through the module path) at 1e-4;
    the mean model's energies differ from the add model's."""
    from mlcg_amd import nn

    cfg = make_cfg(num_blocks=2, rc=12.0, act="ssp", aggr="mean")
    sd = R.random_state_dict(cfg, seed=17)
    b = _small_batch()
    pos64, types, batch, ei = _oracle_inputs(b, 12.0)
    sd64 = R.to_dtype(sd, torch.float64)
    E_ref, F_ref = R.schnet_energy_forces(sd64, cfg, pos64, types, batch, ei, b.n_frames)
    model = make_model(cfg, sd)
    assert model.fused_spec() is None
    data = nn.GradientsOut(model).eval()(b.to_torch("cuda"))
    check(data.out["SchNet"]["energy"], E_ref, 1e-5, "E mean")
    check(data.out["SchNet"]["forces"], F_ref, 1e-5, "F mean")
    E_add, _ = R.schnet_energy_forces(sd64, make_cfg(num_blocks=2, rc=12.0, act="ssp"), pos64,
                                      types, batch, ei, b.n_frames)
    assert float((E_add - E_ref).abs().max()) > 1e-3
    fref64 = torch.from_numpy(b.forces).double()
    loss_ref, _, _, g_ref = R.force_matching_grads(sd64, cfg, pos64, types, batch, ei,
                                                   b.n_frames, fref64)
    model = make_model(cfg, sd)
    gm = nn.GradientsOut(model).train()
    data = gm(b.to_torch("cuda"))
    loss = torch.nn.functional.mse_loss(data.out["SchNet"]["forces"], data.forces)
    loss.backward()
    assert abs(float(loss) - float(loss_ref)) <= 1e-5 * abs(float(loss_ref))
    grads = _param_grads(model)
    for k, gr in g_ref.items():
        assert grads[k] is not None, k
        check(grads[k], gr, 1e-4, k)


def test_compiled_module_path_schnet():
    """A SchNet without a fused pass (mean aggregation) inside torch.compile
    (fullgraph=True): mlcg::direct_energy_forces runs it module by module with
    the position gradient taken inside the operator, as GradientsOut does
    eagerly, so the compiled energies and forces equal the eager ones."""
    import torch._dynamo

    from mlcg_amd import nn

    cfg = make_cfg(num_blocks=2, rc=12.0, act="ssp", aggr="mean")
    sd = R.random_state_dict(cfg, seed=17)
    b = _small_batch()
    gm = nn.GradientsOut(make_model(cfg, sd)).eval()
    ref = gm(b.to_torch("cuda"))
    torch._dynamo.reset()
    out = torch.compile(gm, fullgraph=True, dynamic=True)(b.to_torch("cuda"))
    for key in ("energy", "forces"):
        got, want = out.out["SchNet"][key], ref.out["SchNet"][key]
        assert got.shape == want.shape
        assert torch.allclose(got, want, rtol=1e-6, atol=1e-6), key


@pytest.mark.parametrize("f16", [False, True], ids=["fp32_rows", "fp16_rows"])
def test_gather_bwd_dbar_only_bit_identical(f16):
    """mlcg_cfconv_gather_bwd without ybar (the first block of the force
    sweep, whose input does not depend on the positions) gives the full
    kernel's distance adjoints bit for bit, stored and accumulated."""
    from mlcg_amd import ops

    cfg, sd, b, pos, g, spec, bp = _filter_setup(n_frames=8)
    gen = torch.Generator(device="cpu").manual_seed(7)
    N, P = pos.shape[0], g.pair_capacity
    gagg = torch.randn(N, 128, generator=gen).cuda()
    y = torch.randn(N, 128, generator=gen).cuda()
    W = torch.randn(P, 128, generator=gen).cuda()
    Wd = torch.randn(P, 128, generator=gen).cuda()
    if f16:
        W, Wd = W.half(), Wd.half()
    base = torch.randn(P, generator=gen).cuda()
    for accumulate in (False, True):
        d_full, d_only = base.clone(), base.clone()
        ybar = ops.cfconv_gather_bwd(gagg, y, W, Wd, g, d_full, accumulate=accumulate)
        none = ops.cfconv_gather_bwd(gagg, y, W, Wd, g, d_only, accumulate=accumulate,
                                     want_ybar=False)
        torch.cuda.synchronize()
        assert none is None and ybar is not None
        n = int(g.num_pairs) if hasattr(g, "num_pairs") else P
        assert torch.equal(d_only[:n], d_full[:n]), accumulate
