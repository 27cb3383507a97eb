"""Radial bases on the fused HIP path: the exp-normal basis
(mlcg/nn/radial_basis/exp_normal.py:9-178) and trainable basis parameters
(Gaussian offset/coeff, exp-normal means/betas), against the fp64 oracle.

Tolerances as for the Gaussian path: filter values, energies and forces
rtol 1e-5 (relative to the oracle's norm), parameter gradients rtol 1e-4.
"""

import numpy as np
import pytest
import torch

from oracle import radius as oracle_radius
from oracle import schnet_ref as R
from tests.helpers import check, check_calibrated, make_cfg, make_model, rel_err

pytestmark = pytest.mark.gpu


def _small_batch(n_frames=6, n_beads=14, seed=3):
    from mlcg_amd import synthetic

    rng = np.random.default_rng(seed)
    pos = synthetic.self_avoiding_walk(n_frames, n_beads, rng)
    types = rng.integers(1, 21, size=(n_frames, n_beads))
    forces = rng.standard_normal((n_frames * n_beads, 3)).astype(np.float32)
    return synthetic._flatten(pos, types, seed, forces)


def _oracle_inputs(b, rc):
    ei, _ = oracle_radius.radius_graph(b.pos, rc, b.batch, False, 1000)
    return (torch.from_numpy(b.pos).double(), torch.from_numpy(b.atom_types),
            torch.from_numpy(b.batch), torch.from_numpy(ei))


def _perturbed_sd(cfg, seed):
    """A state dict whose basis parameters are moved off their initial values
    (as after training), so that a kernel reading the wrong ones fails."""
    sd = R.random_state_dict(cfg, seed=seed)
    gen = torch.Generator().manual_seed(seed + 100)
    for k in R.BASIS_KEYS[cfg.basis]:
        t = sd[k]
        sd[k] = t * (1 + 0.05 * (torch.rand(t.shape, generator=gen) * 2 - 1))
    return sd


def _pair_setup(basis, rc=12.0, num_rbf=50, seed=21, rbf_cut="cosine"):
    from mlcg_amd import ops

    cfg = make_cfg(num_blocks=1, rc=rc, num_rbf=num_rbf, basis=basis, rbf_cut=rbf_cut)
    sd = _perturbed_sd(cfg, seed)
    b = _small_batch(n_frames=8, n_beads=20, seed=seed)
    pos = torch.from_numpy(b.pos).cuda()
    g = ops.radius_graph(pos, rc, torch.from_numpy(b.batch).cuda(), max_num_neighbors=1000,
                         with_pairs=True)
    model = make_model(cfg, sd)
    spec = model.fused_spec()
    assert spec is not None
    pij = g.pair_ij.long().cpu()
    p64 = torch.from_numpy(b.pos).double()
    d = (p64[pij[1]] - p64[pij[0]]).norm(dim=1).requires_grad_(True)
    return cfg, R.to_dtype(sd, torch.float64), pos, g, model, spec, d


def _filter_ref(cfg, sd64, d):
    rbf = R.rbf_expand(sd64, cfg, d)
    layers = R._layers(sd64, "interaction_blocks.0.conv.filter_network")
    return R.mlp(rbf, layers, torch.tanh) * R.cosine_cutoff(d, 0.0, cfg.conv_hi).view(-1, 1)


@pytest.mark.parametrize("rbf_cut", ["cosine", "identity"])
def test_expnormal_filter_fwd_matches_torch(rbf_cut):
    from mlcg_amd import ops

    cfg, sd64, pos, g, model, spec, d = _pair_setup("expnormal", rbf_cut=rbf_cut)
    assert spec.filt.basis == ops.BASIS_EXPNORMAL
    blk = model.fused_params().blocks[0]
    W, Wd, dist = ops.filter_fwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2)
    Wr = _filter_ref(cfg, sd64, d)
    Wdr = torch.stack([torch.autograd.grad(Wr[:, f].sum(), d, retain_graph=True)[0]
                       for f in range(128)], dim=1)
    P = g.num_pairs
    print("expnormal W rel", rel_err(W[:P], Wr), "Wd rel", rel_err(Wd[:P], Wdr))
    check(W[:P], Wr.detach(), 1e-5, 'W[:P]')
    check(Wd[:P], Wdr, 1e-5, 'Wd[:P]')


@pytest.mark.parametrize("basis", ["gaussian", "expnormal"])
def test_rbf_param_grad_matches_autograd(basis):
    """d/d(basis parameters) of <Wbar, W> + <Wdbar, dW/dd> from the filter
    backward's pair adjoints and mlcg_rbf_param_grad, against fp64 autograd."""
    from mlcg_amd import ops

    cfg, sd64, pos, g, model, spec, d = _pair_setup(basis)
    blk = model.fused_params().blocks[0]
    P = g.num_pairs
    gen = torch.Generator(device="cuda").manual_seed(4)
    Wbar = torch.zeros(g.pair_capacity, 128, device="cuda")
    Wdbar = torch.zeros(g.pair_capacity, 128, device="cuda")
    Wbar[:P] = torch.randn(P, 128, device="cuda", generator=gen)
    Wdbar[:P] = torch.randn(P, 128, device="cuda", generator=gen)
    dW1, db1, dW2, abar, adbar = ops.filter_bwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2,
                                                Wbar, Wdbar, pair_adjoints=True)
    _, _, dist = ops.filter_fwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2)
    dc, dw = ops.rbf_param_grad(dist, g, spec.filt, blk.W1, abar, adbar)
    # accumulate mode adds on top
    dc2, dw2 = ops.rbf_param_grad(dist, g, spec.filt, blk.W1, abar, adbar,
                                  out=(dc.clone(), dw.clone()))
    keys = R.BASIS_KEYS[basis]
    for k in keys:
        sd64[k] = sd64[k].clone().requires_grad_(True)
    Wr = _filter_ref(cfg, sd64, d)
    wd_term, = torch.autograd.grad((Wr * Wdbar[:P].double().cpu()).sum(), d, create_graph=True)
    obj = (Wr * Wbar[:P].double().cpu()).sum() + wd_term.sum()
    gc, gw = torch.autograd.grad(obj, [sd64[k] for k in keys])
    if basis == "gaussian":
        dw_total = dw.sum()
        dw2_total = dw2.sum()
    else:
        dw_total, dw2_total = dw, dw2
    print(basis, "dcenters rel", rel_err(dc, gc), "dwidths rel", rel_err(dw_total, gw))
    check(dc, gc, 1e-4, 'dc')
    check(dw_total, gw, 1e-4, 'dw_total')
    check(dc2, 2 * gc, 1e-4, 'dc2')
    check(dw2_total, 2 * gw, 1e-4, 'dw2_total')
    # the W1 gradient is unchanged by asking for the pair adjoints
    ref = ops.filter_bwd(pos, g, spec.filt, blk.W1, blk.b1, blk.W2, Wbar, Wdbar)
    assert torch.equal(ref[0], dW1) and torch.equal(ref[1], db1) and torch.equal(ref[2], dW2)


@pytest.mark.parametrize("trainable", [False, True])
def test_expnormal_energy_forces(trainable):
    from mlcg_amd import nn

    cfg = make_cfg(num_blocks=3, rc=12.0, basis="expnormal")
    sd = _perturbed_sd(cfg, seed=5)
    b = _small_batch()
    pos64, types, batch, ei = _oracle_inputs(b, 12.0)
    E_ref, F_ref = R.schnet_energy_forces(R.to_dtype(sd, torch.float64), cfg, pos64, types,
                                          batch, ei, b.n_frames)
    E32, F32 = R.schnet_energy_forces(sd, cfg, pos64.float(), types, batch, ei, b.n_frames)
    model = make_model(cfg, sd, trainable_basis=trainable)
    assert model.fused_spec() is not None
    gm = nn.GradientsOut(model).eval()
    data = gm(b.to_torch("cuda"))
    E = data.out["SchNet"]["energy"]
    F = data.out["SchNet"]["forces"]
    # the exp-normal basis exp(-beta (exp(alpha (lo - d)) - mu)^2), beta = 625,
    # amplifies fp32 rounding of d: the reference's fp32 arithmetic misses the
    # bar here itself (ratio ~1.2), hence the calibrated bound
    check_calibrated(E, E_ref, E32, 1e-5, 'E')
    check_calibrated(F, F_ref, F32, 1e-5, 'F')


@pytest.mark.parametrize("basis,act", [("gaussian", "tanh"), ("expnormal", "tanh"),
                                       ("expnormal", "ssp")])
def test_force_matching_grads_trainable_basis(basis, act):
    """Force-matching parameter gradients (the training step's double
    backward) including the basis parameters."""
    from mlcg_amd import nn

    cfg = make_cfg(num_blocks=3, rc=12.0, act=act, basis=basis)
    sd = _perturbed_sd(cfg, seed=13)
    b = _small_batch()
    pos64, types, batch, ei = _oracle_inputs(b, 12.0)
    fref64 = torch.from_numpy(b.forces).double()
    loss_ref, _, _, g_ref = R.force_matching_grads(R.to_dtype(sd, torch.float64), cfg, pos64,
                                                   types, batch, ei, b.n_frames, fref64,
                                                   trainable_basis=True)
    model = make_model(cfg, sd, trainable_basis=True)
    assert model.fused_spec() is not None
    gm = nn.GradientsOut(model).train()
    data = gm(b.to_torch("cuda"))
    loss = torch.nn.functional.mse_loss(data.out["SchNet"]["forces"], data.forces)
    loss.backward()
    assert abs(float(loss) - float(loss_ref)) <= 1e-5 * abs(float(loss_ref))
    grads = {k: p.grad for k, p in model.named_parameters()}
    for k in R.BASIS_KEYS[basis]:
        assert k in grads and grads[k] is not None, k
        assert grads[k].shape == sd[k].shape
    worst = 0.0
    for k, gr in g_ref.items():
        worst = max(worst, check(grads[k], gr, 1e-4, k))
    print(basis, act, "worst param-grad ratio", worst,
          {k: rel_err(grads[k], g_ref[k]) for k in R.BASIS_KEYS[basis]})


@pytest.mark.parametrize("basis", ["gaussian", "expnormal"])
def test_energy_backward_trainable_basis(basis):
    """First-order path: SchNet.forward then E.backward() reaches the basis."""
    cfg = make_cfg(num_blocks=2, rc=12.0, basis=basis)
    sd = _perturbed_sd(cfg, seed=17)
    b = _small_batch(seed=4)
    pos64, types, batch, ei = _oracle_inputs(b, 12.0)
    sd64 = R.to_dtype(sd, torch.float64)
    for k in R.BASIS_KEYS[basis]:
        sd64[k].requires_grad_(True)
    w = torch.linspace(-1.0, 2.0, b.n_frames, dtype=torch.float64)
    E_ref = R.schnet_energy(sd64, cfg, pos64, types, batch, ei, b.n_frames)
    g_ref = torch.autograd.grad((E_ref * w).sum(), [sd64[k] for k in R.BASIS_KEYS[basis]])
    model = make_model(cfg, sd, trainable_basis=True)
    data = model(b.to_torch("cuda"))
    E = data.out["SchNet"]["energy"]
    (E * w.float().cuda()).sum().backward()
    params = dict(model.named_parameters())
    check(E, E_ref.detach(), 1e-5, 'E')
    for k, gr in zip(R.BASIS_KEYS[basis], g_ref):
        check(params[k].grad, gr, 1e-4, f"{basis} {k}")


def test_pruned_expnormal_basis():
    """build_pruned_from_mask keeps a subset of the functions; the fused path
    runs at the pruned width."""
    from mlcg_amd import nn

    mask = torch.zeros(20, dtype=torch.bool)
    mask[::3] = True
    K = int(mask.sum())
    rbf = nn.ExpNormalBasis.build_pruned_from_mask(nn.CosineCutoff(0.0, 12.0), mask,
                                                   num_rbf=20, trainable=False)
    assert rbf.means.numel() == K and rbf.num_rbf == 20
    cfg = make_cfg(num_blocks=2, rc=12.0, num_rbf=K, basis="expnormal")
    sd = R.random_state_dict(cfg, seed=23)
    means, betas = R.expnormal_params(0.0, 12.0, 20)
    sd["rbf_layer.means"], sd["rbf_layer.betas"] = means[mask], betas[mask]
    # SchNet's constructor resets the basis, which a pruned basis cannot do
    # (its num_rbf stays the unpruned count, as in the reference): build with
    # a full basis of the pruned width, then put the pruned one in
    model = nn.StandardSchNet(nn.ExpNormalBasis(nn.CosineCutoff(0.0, 12.0), num_rbf=K),
                              nn.CosineCutoff(0.0, 12.0), [64], hidden_channels=128,
                              embedding_size=sd["embedding_layer.weight"].shape[0],
                              num_filters=128, num_interactions=2, activation=torch.nn.Tanh())
    model.rbf_layer = rbf
    model.load_state_dict(sd)
    model = model.cuda()
    assert model.fused_spec() is not None and model.fused_spec().filt.num_rbf == K
    b = _small_batch(seed=6)
    pos64, types, batch, ei = _oracle_inputs(b, 12.0)
    E_ref, F_ref = R.schnet_energy_forces(R.to_dtype(sd, torch.float64), cfg, pos64, types,
                                          batch, ei, b.n_frames)
    data = nn.GradientsOut(model).eval()(b.to_torch("cuda"))
    check(data.out["SchNet"]["energy"], E_ref, 1e-5, 'data.out["SchNet"]["energy"]')
    check(data.out["SchNet"]["forces"], F_ref, 1e-5, 'data.out["SchNet"]["forces"]')
