"""Pins the CPU SchNet oracle (oracle/schnet_ref.py) without a GPU.

Each check is chosen so that a plausible slip in the restatement fails it:
  cosine_cutoff     endpoint values of the reference test
                    (tests/unit/nn/test_cutoff.py:27-42) and the closed form
                    at the midpoint
  gaussian_rbf      offsets = linspace, coeff = -0.5/spacing^2
                    (gaussian.py:64-75); e_k(mu_k) == C(mu_k); e_k at one
                    spacing away == exp(-1/2) C
  schnet_energy     a per-node numpy restatement of Appendix-A math on 2- and
                    3-bead frames (catches a swapped gather/scatter direction,
                    a missing residual, a dropped bias); translation,
                    rotation and in-frame permutation invariance; frames are
                    independent; continuity when a pair crosses the cutoff
                    (catches a dropped filter envelope)
  expnormal_rbf     means/betas closed forms (exp_normal.py:80-94); equal to
                    the (pinned) Gaussian of u = exp(alpha (lo - d)) with
                    offsets = means, coeff = -beta; e_k == C where u == mu_k
  forces            central finite differences in fp64; sum_i F_i == 0
  force_matching    the parameter gradient of mean((F - F_ref)^2) against
                    central finite differences along random parameter
                    directions (pins the double backward), with the basis
                    parameters (Gaussian offset/coeff, exp-normal means/betas)
                    trained or fixed
"""

import math

import numpy as np
import pytest
import torch

from oracle import radius as oracle_radius
from oracle import schnet_ref as R

D64 = torch.float64


def _cfg(blocks=2, rc=8.0, act="tanh", rbf_cut="cosine", num_rbf=12, basis="gaussian"):
    return R.SchNetConfig(num_rbf=num_rbf, rbf_lo=0.0, rbf_hi=rc, rbf_cut=rbf_cut,
                          conv_cut="cosine", conv_lo=0.0, conv_hi=rc, act=act,
                          num_blocks=blocks, basis=basis)


def _sd(cfg, seed=0, hidden=128, filters=128):
    return R.to_dtype(R.random_state_dict(cfg, hidden=hidden, filters=filters,
                                          embedding_size=12, seed=seed, bias_scale=0.3), D64)


def _edges(pos, rc, batch):
    ei, _ = oracle_radius.radius_graph(pos.float().numpy(), rc, batch.numpy(), False, 1000)
    return torch.from_numpy(ei)


def _frames(n_frames=3, n=7, seed=0, spread=3.0):
    rng = np.random.default_rng(seed)
    pos = torch.from_numpy(rng.normal(0, spread, (n_frames * n, 3)))
    types = torch.from_numpy(rng.integers(1, 11, n_frames * n))
    batch = torch.arange(n_frames).repeat_interleave(n)
    return pos, types, batch


# --------------------------------------------------------------------------
# elementary pieces

@pytest.mark.parametrize("lo,hi,v0,v1", [(0.0, 5.0, 1.0, 0.0), (5.0, 10.0, 0.0, 0.0)])
def test_cosine_cutoff_endpoints(lo, hi, v0, v1):
    d = torch.linspace(0, 10, 100)
    c = R.cosine_cutoff(d, lo, hi)
    assert float(c[0]) == v0 and float(c[-1]) == v1


def test_cosine_cutoff_closed_form():
    d = torch.tensor([2.5], dtype=D64)
    assert float(R.cosine_cutoff(d, 0.0, 5.0)) == pytest.approx(0.5, abs=1e-15)
    # lower > 0: midpoint of [5, 10] sits at cos(2 pi) -> 1
    assert float(R.cosine_cutoff(torch.tensor([7.5], dtype=D64), 5.0, 10.0)) == pytest.approx(
        1.0, abs=1e-15)
    assert float(R.cosine_cutoff(torch.tensor([6.25], dtype=D64), 5.0, 10.0)) == pytest.approx(
        0.5, abs=1e-15)


def test_gaussian_params_and_values():
    off, coeff = R.gaussian_params(0.0, 20.0, 50, D64)
    assert torch.allclose(off, torch.arange(50, dtype=D64) * (20.0 / 49))
    spacing = 20.0 / 49
    assert float(coeff) == pytest.approx(-0.5 / spacing ** 2, rel=1e-6)
    cut = R.Cutoff("cosine", 0.0, 20.0)
    e = R.gaussian_rbf(off, off, coeff, cut)  # e[k, k] = C(mu_k)
    assert torch.allclose(torch.diagonal(e), R.cosine_cutoff(off, 0.0, 20.0))
    e1 = R.gaussian_rbf(off[:-1] + spacing, off, coeff, R.Cutoff("identity", 0.0, 20.0))
    ks = torch.arange(49)
    assert torch.allclose(e1[ks, ks], torch.full((49,), math.exp(-0.5), dtype=D64), rtol=1e-6)


@pytest.mark.parametrize("lo,hi,K", [(0.0, 5.0, 8), (0.5, 12.0, 50)])
def test_expnormal_params_and_values(lo, hi, K):
    means, betas = R.expnormal_params(lo, hi, K, D64)
    start = math.exp(lo - hi)
    assert float(means[0]) == pytest.approx(start, rel=1e-6)
    assert float(means[-1]) == pytest.approx(1.0, rel=1e-7)
    assert torch.allclose(means[1:] - means[:-1],
                          torch.full((K - 1,), (1 - start) / (K - 1), dtype=D64), rtol=1e-5)
    assert torch.allclose(betas, torch.full((K,), (2.0 / K * (1 - start)) ** -2, dtype=D64),
                          rtol=1e-6)
    alpha = R.expnormal_alpha(lo, hi)
    assert alpha == pytest.approx(5.0 / (hi - lo))
    cut = R.Cutoff("cosine", lo, hi)
    gen = torch.Generator().manual_seed(0)
    d = lo + (hi - lo) * torch.rand(40, dtype=D64, generator=gen)
    b = 3.0 + torch.rand(1, dtype=D64, generator=gen)
    e = R.expnormal_rbf(d, means, b.expand(K), alpha, lo, cut)
    # a Gaussian in u = exp(alpha (lo - d)) with the means as offsets
    u = torch.exp(alpha * (lo - d))
    g = R.gaussian_rbf(u, means, -b, R.Cutoff("identity", 0.0, 1.0))
    assert torch.allclose(e, g * cut(d).unsqueeze(-1), rtol=1e-12, atol=0)
    # e_k == C(d_k) where u(d_k) == mu_k, i.e. d_k = lo - ln(mu_k) / alpha
    dk = lo - torch.log(means) / alpha
    ek = R.expnormal_rbf(dk, means, betas, alpha, lo, cut)
    assert torch.allclose(torch.diagonal(ek), cut(dk), rtol=1e-12, atol=1e-15)


# --------------------------------------------------------------------------
# per-node numpy restatement of the math (no index_add, no edge lists)

def _np_act(name):
    if name == "tanh":
        return np.tanh
    return lambda x: np.log1p(np.exp(x)) - math.log(2.0)


def _np_energy(sd, cfg, pos, types):
    """Energy of ONE frame: loops over receivers i and senders j != i."""
    act = _np_act(cfg.act)
    s = {k: v.numpy() for k, v in sd.items()}
    pos = pos.numpy()
    types = types.numpy()
    n = pos.shape[0]
    rc = cfg.conv_hi
    if cfg.basis == "gaussian":
        off, coeff = s["rbf_layer.offset"], float(s["rbf_layer.coeff"])

        def basis(d):
            return np.exp(coeff * (d - off) ** 2)
    else:
        means, betas = s["rbf_layer.means"], s["rbf_layer.betas"]
        alpha = 5.0 / (cfg.rbf_hi - cfg.rbf_lo)

        def basis(d):
            return np.exp(-betas * (math.exp(-alpha * (d - cfg.rbf_lo)) - means) ** 2)

    def cosc(d):
        return 0.5 * (math.cos(d * math.pi / rc) + 1.0) if d < rc else 0.0

    x = s["embedding_layer.weight"][types].copy()
    for b in range(cfg.num_blocks):
        p = f"interaction_blocks.{b}"
        W1 = s[f"{p}.conv.filter_network.layers.0.weight"]
        b1 = s[f"{p}.conv.filter_network.layers.0.bias"]
        W2 = s[f"{p}.conv.filter_network.layers.2.weight"]
        y = x @ s[f"{p}.conv.lin1.weight"].T
        agg = np.zeros_like(y)
        for i in range(n):
            for j in range(n):
                if i == j:
                    continue
                d = float(np.linalg.norm(pos[j] - pos[i]))
                if not np.float32(d) < np.float32(rc):
                    continue
                crbf = cosc(d) if cfg.rbf_cut == "cosine" else 1.0
                g = basis(d) * crbf
                w = W2 @ act(W1 @ g + b1) * cosc(d)
                agg[i] += y[j] * w
        z = agg @ s[f"{p}.conv.lin2.weight"].T + s[f"{p}.conv.lin2.bias"]
        x = x + act(z) @ s[f"{p}.lin.weight"].T + s[f"{p}.lin.bias"]
    h = act(x @ s["output_network.layers.0.weight"].T + s["output_network.layers.0.bias"])
    o = h @ s["output_network.layers.2.weight"].T
    return float(o.sum())


@pytest.mark.parametrize("basis", ["gaussian", "expnormal"])
@pytest.mark.parametrize("act", ["tanh", "ssp"])
@pytest.mark.parametrize("n_beads", [2, 3, 5])
def test_energy_matches_per_node_restatement(act, n_beads, basis):
    cfg = _cfg(blocks=2, rc=6.0, act=act, basis=basis)
    sd = _sd(cfg, seed=n_beads)
    rng = np.random.default_rng(n_beads)
    pos = torch.from_numpy(rng.normal(0, 2.0, (n_beads, 3)))
    if n_beads == 3:
        pos[2] = torch.tensor([40.0, 0.0, 0.0])  # isolated bead
    types = torch.from_numpy(rng.permutation(np.arange(1, 11))[:n_beads].copy())
    batch = torch.zeros(n_beads, dtype=torch.long)
    E = R.schnet_energy(sd, cfg, pos, types, batch, _edges(pos, 6.0, batch), 1)
    assert float(E[0]) == pytest.approx(_np_energy(sd, cfg, pos, types), rel=1e-12)


def test_invariances_and_frame_independence():
    cfg = _cfg(blocks=3, rc=8.0)
    sd = _sd(cfg, seed=1)
    pos, types, batch = _frames(3, 8, seed=2)
    E = R.schnet_energy(sd, cfg, pos, types, batch, _edges(pos, 8.0, batch), 3)
    # translation (per frame) and a rotation
    q, _ = torch.linalg.qr(torch.randn(3, 3, dtype=D64, generator=torch.Generator().manual_seed(4)))
    pos2 = pos @ q.T + torch.randn(3, 1, dtype=D64).repeat_interleave(8, 0)
    E2 = R.schnet_energy(sd, cfg, pos2, types, batch, _edges(pos2, 8.0, batch), 3)
    assert torch.allclose(E, E2, rtol=1e-10)
    # in-frame permutation of beads together with their types
    perm = torch.cat([torch.randperm(8, generator=torch.Generator().manual_seed(b)) + 8 * b
                      for b in range(3)])
    E3 = R.schnet_energy(sd, cfg, pos[perm], types[perm], batch,
                         _edges(pos[perm], 8.0, batch), 3)
    assert torch.allclose(E, E3, rtol=1e-10)
    # each frame alone gives the same energy
    for b in range(3):
        sl = slice(8 * b, 8 * b + 8)
        zb = torch.zeros(8, dtype=torch.long)
        Eb = R.schnet_energy(sd, cfg, pos[sl], types[sl], zb, _edges(pos[sl], 8.0, zb), 1)
        assert float(Eb[0]) == pytest.approx(float(E[b]), rel=1e-12)


def test_energy_continuous_across_cutoff():
    cfg = _cfg(blocks=2, rc=5.0, rbf_cut="identity")
    sd = _sd(cfg, seed=3)
    types = torch.tensor([1, 2])
    batch = torch.zeros(2, dtype=torch.long)
    Es = []
    for x in (5.0 - 1e-6, 5.0 + 1e-6):
        pos = torch.tensor([[0.0, 0.0, 0.0], [x, 0.0, 0.0]], dtype=D64)
        Es.append(float(R.schnet_energy(sd, cfg, pos, types, batch,
                                        _edges(pos, 5.0, batch), 1)[0]))
    assert abs(Es[0] - Es[1]) < 1e-9


@pytest.mark.parametrize("act", ["tanh", "ssp"])
def test_forces_finite_differences(act):
    cfg = _cfg(blocks=2, rc=7.0, act=act)
    sd = _sd(cfg, seed=5)
    pos, types, batch = _frames(2, 6, seed=6, spread=2.5)
    ei = _edges(pos, 7.0, batch)
    E, F = R.schnet_energy_forces(sd, cfg, pos, types, batch, ei, 2)
    h = 1e-5
    Ffd = torch.zeros_like(pos)
    for n in range(pos.shape[0]):
        for c in range(3):
            pp, pm = pos.clone(), pos.clone()
            pp[n, c] += h
            pm[n, c] -= h
            Ep = R.schnet_energy(sd, cfg, pp, types, batch, ei, 2).sum()
            Em = R.schnet_energy(sd, cfg, pm, types, batch, ei, 2).sum()
            Ffd[n, c] = -(Ep - Em) / (2 * h)
    assert torch.allclose(F, Ffd, rtol=1e-6, atol=1e-8)
    for b in range(2):
        assert torch.allclose(F[batch == b].sum(0), torch.zeros(3, dtype=D64), atol=1e-10)


@pytest.mark.parametrize("act,basis,trainable", [
    ("tanh", "gaussian", False), ("ssp", "gaussian", False), ("tanh", "gaussian", True),
    ("tanh", "expnormal", True), ("ssp", "expnormal", True), ("tanh", "expnormal", False)])
def test_force_matching_grads_finite_differences(act, basis, trainable):
    cfg = _cfg(blocks=2, rc=7.0, act=act, basis=basis)
    sd = _sd(cfg, seed=7)
    pos, types, batch = _frames(2, 6, seed=8, spread=2.5)
    ei = _edges(pos, 7.0, batch)
    fref = torch.randn(pos.shape, dtype=D64, generator=torch.Generator().manual_seed(9))
    loss, _, _, grads = R.force_matching_grads(sd, cfg, pos, types, batch, ei, 2, fref,
                                               trainable_basis=trainable)
    assert all(k in grads for k in R.BASIS_KEYS[basis]) == trainable
    gen = torch.Generator().manual_seed(10)
    names = list(grads)
    for trial in range(3):
        direction = {k: torch.randn(grads[k].shape, dtype=D64, generator=gen) for k in names}
        ana = sum(float((grads[k] * direction[k]).sum()) for k in names)
        h = 1e-6

        def loss_at(sign):
            sd2 = dict(sd)
            for k in names:
                sd2[k] = sd[k] + sign * h * direction[k]
            _, F = R.schnet_energy_forces(sd2, cfg, pos, types, batch, ei, 2)
            return float(R.force_mse(F, fref))

        fd = (loss_at(1.0) - loss_at(-1.0)) / (2 * h)
        assert ana == pytest.approx(fd, rel=1e-6, abs=1e-10), trial
    # every parameter gets a non-trivial gradient (embedding rows of unused
    # types excepted)
    for k in names:
        if k != "embedding_layer.weight":
            assert float(grads[k].abs().max()) > 0, k


@pytest.mark.parametrize("basis", ["gaussian", "expnormal"])
def test_energy_basis_gradients_finite_differences(basis):
    """dE/d(basis parameters) by autograd through the oracle against central
    differences (the first-order path a trainable basis takes)."""
    cfg = _cfg(blocks=2, rc=7.0, basis=basis)
    sd = _sd(cfg, seed=11)
    pos, types, batch = _frames(2, 6, seed=12, spread=2.5)
    ei = _edges(pos, 7.0, batch)
    keys = R.BASIS_KEYS[basis]
    w = torch.tensor([0.7, -1.3], dtype=D64)
    sd2 = dict(sd)
    for k in keys:
        sd2[k] = sd[k].clone().requires_grad_(True)
    E = R.schnet_energy(sd2, cfg, pos, types, batch, ei, 2)
    grads = torch.autograd.grad((E * w).sum(), [sd2[k] for k in keys])
    gen = torch.Generator().manual_seed(13)
    for k, g in zip(keys, grads):
        assert float(g.abs().max()) > 0, k
        v = torch.randn(sd[k].shape, dtype=D64, generator=gen)
        h = 1e-6 * max(1.0, float(sd[k].abs().max()))

        def e_at(sign):
            sd3 = dict(sd)
            sd3[k] = sd[k] + sign * h * v
            return float((R.schnet_energy(sd3, cfg, pos, types, batch, ei, 2) * w).sum())

        fd = (e_at(1.0) - e_at(-1.0)) / (2 * h)
        assert float((g * v).sum()) == pytest.approx(fd, rel=1e-6, abs=1e-9), k


def test_golden_fixture_reproduced():
    """The committed SchNet fixture (tests/golden/make_golden.py) is what the
    oracle computes today."""
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", "schnet_small.pt")
    g = torch.load(path, weights_only=True)
    cfg = R.SchNetConfig(**g["cfg"])
    sd = g["state_dict"]
    E, F = R.schnet_energy_forces(sd, cfg, g["pos"], g["types"], g["batch"], g["edge_index"],
                                  int(g["n_frames"]))
    assert torch.allclose(E, g["energy"], rtol=1e-12, atol=0)
    assert torch.allclose(F, g["forces"], rtol=1e-12, atol=1e-14)
    loss, _, _, grads = R.force_matching_grads(sd, cfg, g["pos"], g["types"], g["batch"],
                                               g["edge_index"], int(g["n_frames"]),
                                               g["forces_ref"])
    assert float(loss) == pytest.approx(float(g["loss"]), rel=1e-12)
    for k, v in grads.items():
        assert torch.allclose(v, g["grads"][k], rtol=1e-10, atol=1e-14), k


def test_chunked_force_matching_equals_whole_batch():
    """force_matching_grads_chunked (frame chunks, weighted by chunk size)
    gives the whole-batch loss, energies, forces and gradients: catches a
    chunk weight of 1/chunks instead of N_c/N, or an edge list not shifted to
    the chunk's node numbering."""
    cfg = _cfg(blocks=2, rc=8.0)
    sd = _sd(cfg, seed=3)
    pos, types, batch = _frames(n_frames=5, n=6, seed=4, spread=2.5)
    # ragged frames: drop two beads of frame 1
    keep = torch.ones(pos.shape[0], dtype=torch.bool)
    keep[7:9] = False
    pos, types, batch = pos[keep], types[keep], batch[keep]
    ei = _edges(pos, 8.0, batch)
    fref = torch.from_numpy(np.random.default_rng(5).normal(0, 1, (pos.shape[0], 3)))
    whole = R.force_matching_grads(sd, cfg, pos, types, batch, ei, 5, fref)
    for chunk in (1, 2, 3):
        part = R.force_matching_grads_chunked(sd, cfg, pos, types, batch, ei, 5, fref,
                                              frames_per_chunk=chunk)
        assert float(part[0]) == pytest.approx(float(whole[0]), rel=1e-12)
        assert torch.allclose(part[1], whole[1], rtol=1e-12, atol=1e-14)
        assert torch.allclose(part[2], whole[2], rtol=1e-12, atol=1e-14)
        for k, v in whole[3].items():
            assert torch.allclose(part[3][k], v, rtol=1e-10, atol=1e-14), (chunk, k)


@pytest.mark.parametrize("aggr", ["add", "mean"])
def test_aggregate_matches_per_receiver_loops(aggr):
    """The oracle's CFConv aggregation (PyG MessagePassing aggr="add" /
    "mean") against explicit per-receiver loops over the edge list, with a
    receiver that gets no message (zero in both) and repeated receivers."""
    g = torch.Generator().manual_seed(5)
    n, F = 7, 4
    index = torch.tensor([0, 0, 3, 2, 3, 3, 6, 0, 2, 5])
    msg = torch.randn(index.numel(), F, generator=g, dtype=torch.float64)
    got = R.aggregate(msg, index, n, aggr)
    for t in range(n):
        rows = [msg[e] for e in range(index.numel()) if int(index[e]) == t]
        want = torch.zeros(F, dtype=torch.float64)
        for r in rows:
            want = want + r
        if aggr == "mean" and rows:
            want = want / len(rows)
        assert torch.allclose(got[t], want, rtol=0, atol=1e-15), t
    assert torch.equal(got[1], torch.zeros(F, dtype=torch.float64))  # no messages
    with pytest.raises(ValueError):
        R.aggregate(msg, index, n, "max")
