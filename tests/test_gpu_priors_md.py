"""HIP priors, BAOAB integrator and the captured MD step against the CPU
oracles (oracle/priors_ref.py, oracle/langevin_ref.py).

Tolerances: fp32 energies and forces within 1e-5
of the fp64 oracle per element (tests.helpers.check: rtol 1e-5 of the element,
or 1e-6 of the tensor's largest element).
"""

import math

import numpy as np
import pytest
import torch

from oracle import langevin_ref as L
from oracle import priors_ref as P
from tests.helpers import check, rel_err

pytestmark = pytest.mark.gpu

KINDS = ["bonds", "angles", "dihedrals", "repulsion"]


def _chain_batch(n_frames, n_beads, seed=5):
    from mlcg_amd import synthetic

    rng = np.random.default_rng(seed)
    pos = synthetic.self_avoiding_walk(n_frames, n_beads, rng)
    return torch.from_numpy(pos.reshape(-1, 3))


def _param_matrix(kind, params):
    if kind in ("bonds", "angles"):
        return torch.stack([params["x0"], params["k"], params["V0"]], 1)
    if kind == "dihedrals":
        return torch.cat([params["v_0"][:, None], params["k1s"], params["k2s"]], 1)
    return params["sigma"][:, None]


def _params(kind, M, seed=3):
    g = torch.Generator().manual_seed(seed)
    if kind == "bonds":
        return {"x0": 3.8 + 0.1 * torch.randn(M, generator=g), "k": torch.full((M,), 100.0),
                "V0": torch.zeros(M)}
    if kind == "angles":
        return {"x0": torch.full((M,), math.cos(math.radians(100.0))),
                "k": 5.0 + torch.rand(M, generator=g), "V0": 0.1 * torch.rand(M, generator=g)}
    if kind == "dihedrals":
        return {"v_0": torch.rand(M, generator=g), "k1s": 0.5 * torch.randn(M, 3, generator=g),
                "k2s": 0.5 * torch.randn(M, 3, generator=g)}
    return {"sigma": torch.full((M,), 4.0)}


@pytest.mark.parametrize("kind", KINDS)
def test_prior_kernel_vs_oracle(kind):
    from mlcg_amd import ops

    n_frames, n = 6, 268
    pos = _chain_batch(n_frames, n)
    mapping, mb = P.chain_topology(n_frames, n)[kind]
    params = _params(kind, mapping.shape[1])
    E_ref, F_ref = P.prior_energy_forces(kind, pos.double(), mapping, mb, n_frames,
                                         {k: v.double() for k, v in params.items()})
    g = ops.prior_graph(mapping.cuda(), mb.cuda(), pos.shape[0], n_frames)
    E, F = ops.prior_energy_forces(ops.PRIOR_KIND[kind], 3, pos.cuda(), g,
                                   _param_matrix(kind, params).cuda())
    print(kind, "E rel", rel_err(E, E_ref), "F rel", rel_err(F, F_ref))
    check(E, E_ref, 1e-5, 'E')
    check(F, F_ref, 1e-5, 'F')
    # accumulate mode adds onto an existing force array
    F0 = torch.ones_like(F)
    _, F2 = ops.prior_energy_forces(ops.PRIOR_KIND[kind], 3, pos.cuda(), g,
                                    _param_matrix(kind, params).cuda(), forces=F0)
    assert torch.allclose(F2, F + 1.0, rtol=1e-6, atol=1e-6)


def test_repulsion_direct_forces_bit_identical_to_slot_forces():
    """The repulsion prior's per-bead direct forces (mlcg_prior_pair_records +
    mlcg_prior_repulsion_forces) equal the slot-force path (mlcg_prior_terms
    with slot forces + mlcg_prior_gather_forces) bit for bit at config-5 size,
    set and accumulate modes, and follow an in-place change of the parameter
    matrix (the cached records are rebuilt for the new version)."""
    from mlcg_amd import _lib, ops

    n_frames, n = 100, 268
    pos = _chain_batch(n_frames, n, seed=11).cuda()
    mapping, mb = P.chain_topology(n_frames, n)["repulsion"]
    M = mapping.shape[1]
    g = ops.prior_graph(mapping.cuda(), mb.cuda(), pos.shape[0], n_frames)
    gen = torch.Generator().manual_seed(4)
    params = (3.5 + torch.rand(M, 1, generator=gen)).cuda()
    kind = ops.PRIOR_KIND["repulsion"]

    def slot_path(F0=None):
        energy, slot_f = ops.prior_terms(kind, 0, pos, g, params)
        out = torch.empty(n_frames * n, 3, device="cuda") if F0 is None else F0.clone()
        _lib.call("mlcg_prior_gather_forces", _lib.ptr(slot_f), _lib.ptr(g.bead_ptr),
                  _lib.ptr(g.bead_slots), g.num_nodes, int(F0 is not None), _lib.ptr(out),
                  _lib.stream_handle(pos.device))
        return ops.segment_sum(energy, g.seg_ptr), out

    for rnd in range(2):
        E_ref, F_ref = slot_path()
        E, F = ops.prior_energy_forces(kind, 0, pos, g, params)
        assert torch.equal(E, E_ref) and torch.equal(F, F_ref), rnd
        F0 = torch.randn(n_frames * n, 3, device="cuda")
        _, Fa_ref = slot_path(F0)
        _, Fa = ops.prior_energy_forces(kind, 0, pos, g, params, forces=F0.clone())
        assert torch.equal(Fa, Fa_ref), rnd
        print("round", rnd, "max|F|", float(F.abs().max()))
        params.mul_(1.05)  # new version: the records must be made again


def _stats_tables():
    bonds = {(a, b): {"x_0": 3.8 + 0.01 * (a + b), "k": 100.0 - a} for a in range(1, 6)
             for b in range(1, 6)}
    angles = {(a, b, c): {"x_0": math.cos(math.radians(95 + a + c)), "k": 4.0 + 0.1 * b}
              for a in range(1, 6) for b in range(1, 6) for c in range(1, 6)}
    dih = {}
    for a in range(1, 3):
        for b in range(1, 6):
            for c in range(1, 6):
                for d in range(1, 3):
                    dih[(a, b, c, d)] = {
                        "k1s": {f"k1_{i}": 0.1 * i * (a - d + 0.5) for i in (1, 2, 3)},
                        "k2s": {f"k2_{i}": 0.2 / i * (b - c + 0.3) for i in (1, 2, 3)},
                        "v_0": 0.05 * (a + b)}
    rep = {(a, b): {"sigma": 3.5 + 0.1 * (a + b)} for a in range(1, 6) for b in range(1, 6)}
    return bonds, angles, dih, rep


def _md_config(n_frames=4, n_beads=20, seed=9, with_rep=True):
    from mlcg_amd.data import AtomicData

    rng = np.random.default_rng(seed)
    from mlcg_amd import synthetic

    pos3 = synthetic.self_avoiding_walk(n_frames, n_beads, rng)
    confs = []
    for f in range(n_frames):
        types = torch.from_numpy(rng.integers(1, 6, n_beads))
        types[::7] = 1  # dihedral table covers end types 1..2
        types[0] = types[-1] = 1
        topo = P.chain_topology(1, n_beads)
        nl = {}
        for name in ("bonds", "angles", "dihedrals") + (("repulsion",) if with_rep else ()):
            nl[name] = {"index_mapping": topo[name][0], "order": topo[name][0].shape[0]}
        confs.append(AtomicData(pos=torch.from_numpy(pos3[f]), atom_types=types,
                                masses=torch.full((n_beads,), 12.0 / 418.4),
                                n_atoms=torch.tensor([n_beads]), neighbor_list=nl))
    return confs


def _dihedral_types_ok(data):
    m = data.neighbor_list["dihedrals"]["index_mapping"]
    t = data.atom_types
    return bool(((t[m[0]] <= 2) & (t[m[3]] <= 2)).all())


def test_prior_modules_sumout_and_static():
    """Module API: every prior through GradientsOut equals the oracle; SumOut
    total equals the sum of its parts (tests/unit/nn/test_outs.py:134-166);
    the condensed static priors give the same energies and forces."""
    from mlcg_amd import nn
    from mlcg_amd.data.atomic_data import collate
    from mlcg_amd.simulation import condense_all_priors_for_simulation

    bonds, angles, dih, rep = _stats_tables()
    confs = _md_config()
    # keep only dihedrals whose end types are in the table's range
    for c in confs:
        m = c.neighbor_list["dihedrals"]["index_mapping"]
        keep = (c.atom_types[m[0]] <= 2) & (c.atom_types[m[3]] <= 2)
        c.neighbor_list["dihedrals"]["index_mapping"] = m[:, keep]
    priors = torch.nn.ModuleDict({
        "bonds": nn.GradientsOut(nn.HarmonicBonds(bonds)),
        "angles": nn.GradientsOut(nn.HarmonicAngles(angles)),
        "dihedrals": nn.GradientsOut(nn.Dihedral(dih, n_degs=3)),
        "repulsion": nn.GradientsOut(nn.Repulsion(rep))})
    model = nn.SumOut(priors).cuda()
    data = collate(confs).to("cuda")
    out = model(data)
    total_E = torch.zeros_like(out.out["energy"])
    total_F = torch.zeros_like(out.out["forces"])
    for name, gm in priors.items():
        e = out.out[name]["energy"]
        f = out.out[name]["forces"]
        total_E += e
        total_F += f
        # against the oracle with the reference's type-table gather
        prior = gm.model
        pp = {k: v.double().cpu() for k, v in prior.data2parameters(data).items()}
        if name == "repulsion":
            pp = {"sigma": pp["sigma"]}
        nlm = data.neighbor_list[name]
        E_ref, F_ref = P.prior_energy_forces(name, data.pos.double().cpu(),
                                             nlm["index_mapping"].cpu(),
                                             nlm["mapping_batch"].cpu(), 4, pp)
        check(e, E_ref, 1e-5, name)
        check(f, F_ref, 1e-5, name)
    # the one-launch sum adds the parts in the loop's order: bit for bit
    assert torch.equal(out.out["energy"], total_E)
    assert torch.equal(out.out["forces"], total_F)
    # generic autograd route: forward energy, then grad wrt pos
    d2 = collate(confs).to("cuda")
    d2.pos.requires_grad_(True)
    d2 = priors["dihedrals"].model(d2)
    (gpos,) = torch.autograd.grad(d2.out["dihedrals"]["energy"].sum(), d2.pos)
    check(-gpos, out.out["dihedrals"]["forces"], 1e-6, '-gpos')
    # static specialisation
    sp, sconfs = condense_all_priors_for_simulation(model.cpu(), confs)
    sp = sp.cuda()
    sdata = collate(sconfs).to("cuda")
    sout = sp(sdata)
    assert torch.allclose(sout.out["energy"], out.out["energy"], rtol=1e-6, atol=1e-5)
    assert torch.allclose(sout.out["forces"], out.out["forces"], rtol=1e-6, atol=1e-5)


def test_baoab_kernel_vs_oracle():
    from mlcg_amd import ops

    rng = np.random.default_rng(11)
    n = 1000
    x = torch.from_numpy(rng.normal(size=(n, 3)).astype(np.float32))
    v = torch.from_numpy(rng.normal(size=(n, 3)).astype(np.float32))
    F = torch.from_numpy(rng.normal(size=(n, 3)).astype(np.float32))
    Fn = torch.from_numpy(rng.normal(size=(n, 3)).astype(np.float32))
    m = torch.from_numpy(rng.uniform(0.02, 0.04, n).astype(np.float32))
    bmr = torch.sqrt(1.0 / (L.beta_of(300.0) * m))
    xi = torch.from_numpy(rng.normal(size=(n, 3)).astype(np.float32))
    vs, ns = L.constants(0.004, 1.0)
    xr, vr = L.baoa(x.double(), v.double(), F.double(), m.double(), bmr.double(), 0.004, vs,
                    ns, xi.double())
    vr = L.b(vr, Fn.double(), m.double(), 0.004)
    xg, vg = x.cuda(), v.cuda()
    step = torch.zeros(1, dtype=torch.int64, device="cuda")
    ops.langevin_baoa(xg, vg, F.cuda(), m.cuda(), bmr.cuda(), 0.004, vs, ns, 7, step=step,
                      noise=xi.cuda())
    ops.langevin_b(vg, Fn.cuda(), m.cuda(), 0.004, step=step)
    check(xg, xr, 1e-6, 'xg')
    check(vg, vr, 1e-6, 'vg')
    assert int(step.item()) == 1


def test_philox_normals_moments_and_streams():
    from mlcg_amd import ops

    z = ops.philox_normals(1234, 0, 400_000, "cuda").double()
    assert abs(float(z.mean())) < 5e-3
    assert abs(float(z.var()) - 1.0) < 1e-2
    assert abs(float((z ** 3).mean())) < 1e-2
    assert abs(float((z ** 4).mean()) - 3.0) < 3e-2
    # components uncorrelated, steps and seeds give different streams
    c = torch.corrcoef(z[:, :3].t().float())
    assert float((c - torch.eye(3, device="cuda")).abs().max()) < 1e-2
    z1 = ops.philox_normals(1234, 1, 1000, "cuda")
    z2 = ops.philox_normals(1235, 0, 1000, "cuda")
    assert not torch.equal(z1, z[:1000].float()) and not torch.equal(z2, z[:1000].float())
    assert torch.equal(ops.philox_normals(1234, 0, 1000, "cuda"), z[:1000].float())


def test_langevin_thermostat_equipartition():
    """Soft harmonic bonds only, 256 chains of 12 beads at 300 K: after
    equilibration the kinetic energy per degree of freedom is 1/(2 beta)
    (the Maxwell-Boltzmann check of tests/unit/simulation/
    test_simulation.py:451-472, here through the dynamics)."""
    from mlcg_amd import nn
    from mlcg_amd.simulation import LangevinSimulation

    bonds = {(a, b): {"x_0": 3.8, "k": 5.0} for a in range(1, 6) for b in range(1, 6)}
    confs = _md_config(n_frames=256, n_beads=12, with_rep=False)
    for c in confs:
        for k in ("angles", "dihedrals"):
            c.neighbor_list.pop(k)
    model = nn.SumOut(torch.nn.ModuleDict({"bonds": nn.GradientsOut(nn.HarmonicBonds(bonds))}))
    beta = L.beta_of(300.0)
    sim = LangevinSimulation(friction=10.0, dt=0.004, n_timesteps=3000, save_interval=1000,
                             random_seed=3, capture=True)
    sim.attach_model_and_configurations(model, confs, beta)
    sim.simulate()
    v = sim.final_data.velocities.double()
    m = sim.final_data.masses.double()
    ke_per_dof = float((0.5 * m[:, None] * v * v).mean())
    assert ke_per_dof == pytest.approx(0.5 / beta, rel=0.08)


def test_sumout_one_launch_sum_matches_loop_with_gradients():
    """SumOut over GradientsOut models adds their outputs in one launch: the
    totals and, in training, every parameter gradient through the summed
    forces equal those of the reference's running-sum loop bit for bit."""
    from mlcg_amd import nn
    from mlcg_amd.data.atomic_data import collate
    from oracle import schnet_ref as R
    from tests.helpers import make_cfg, make_model

    bonds, _, _, _ = _stats_tables()
    cfg = make_cfg(num_blocks=2, rc=20.0)
    sd = R.random_state_dict(cfg, seed=41)
    confs = _md_config()
    runs = []
    for fused in (True, False):
        schnet = make_model(cfg, sd).train()
        model = nn.SumOut(torch.nn.ModuleDict({
            "SchNet": nn.GradientsOut(schnet),
            "bonds": nn.GradientsOut(nn.HarmonicBonds(bonds))})).cuda().train()
        if not fused:
            model._outputs_independent = lambda: False
        data = collate(confs).to("cuda")
        out = model(data)
        loss = (out.out["forces"] ** 2).mean() + out.out["energy"].sum()
        loss.backward()
        runs.append((out.out["energy"].detach(), out.out["forces"].detach(),
                     [p.grad.clone() for p in schnet.parameters() if p.grad is not None]))
    (e1, f1, g1), (e2, f2, g2) = runs
    assert torch.equal(e1, e2) and torch.equal(f1, f2)
    assert len(g1) == len(g2) and len(g1) > 0
    for a, c in zip(g1, g2):
        assert torch.equal(a, c)


def test_radius_graph_capacity_mode():
    from mlcg_amd import ops, synthetic

    b = synthetic.config2(n_frames=32)
    pos = torch.from_numpy(b.pos).cuda()
    batch = torch.from_numpy(b.batch).cuda()
    g = ops.radius_graph(pos, 20.0, batch, False, 1000, with_pairs=True, n_frames=32)
    gc = ops.radius_graph(pos, 20.0, batch, False, 1000, with_pairs=True, n_frames=32,
                          capacity=g.num_edges + 100)
    E, P_ = g.num_edges, g.num_pairs
    assert int(gc.flags.item()) == 0
    assert torch.equal(gc.edge_index[:, :E], g.edge_index)
    assert torch.equal(gc.rowptr, g.rowptr)
    assert torch.equal(gc.pair_ij[:, :P_], g.pair_ij)
    assert torch.equal(gc.eid2pair[:E], g.eid2pair)
    assert int(gc.n_pairs_dev.item()) == P_
    small = ops.radius_graph(pos, 20.0, batch, False, 1000, with_pairs=True, n_frames=32,
                             capacity=E // 2)
    assert int(small.flags.item()) & 2
    live = int(small.rowptr[-1].item())
    assert live <= E // 2
    # every edge the clamped CSR holds names a stored pair (pair 0 for the
    # lower copies of pairs that fell past the pair capacity)
    e2p = small.eid2pair[:live]
    assert int(e2p.min().item()) >= 0 and int(e2p.max().item()) < (E // 2) // 2


def test_md_step_captured_matches_eager():
    """SchNet (config-2 architecture, rc 20) + priors on 268-bead chains: the
    hipGraph-captured BAOAB step replays give the same trajectory as the eager
    loop (every replay checked through the saved frames)."""
    from mlcg_amd import nn
    from mlcg_amd.simulation import LangevinSimulation

    bonds, angles, dih, rep = _stats_tables()

    def build():
        torch.manual_seed(0)
        rbf = nn.GaussianBasis(nn.CosineCutoff(0, 20.0), num_rbf=50)
        schnet = nn.StandardSchNet(rbf, nn.CosineCutoff(0, 20.0), [64], 128, 100, 128, 3,
                                   torch.nn.Tanh())
        return nn.SumOut(torch.nn.ModuleDict({
            "SchNet": nn.GradientsOut(schnet),
            "bonds": nn.GradientsOut(nn.HarmonicBonds(bonds)),
            "angles": nn.GradientsOut(nn.HarmonicAngles(angles)),
            "repulsion": nn.GradientsOut(nn.Repulsion(rep))}))

    confs = _md_config(n_frames=3, n_beads=60)
    for c in confs:
        c.neighbor_list.pop("dihedrals")
    trajs = []
    for capture in (False, True):
        sim = LangevinSimulation(friction=1.0, dt=0.004, n_timesteps=12, save_interval=1,
                                 random_seed=21, capture=capture, save_energies=True)
        sim.attach_model_and_configurations(build(), [c.clone() for c in confs],
                                            L.beta_of(300.0))
        trajs.append((sim.simulate(), sim.simulated_potential))
    (x0, e0), (x1, e1) = trajs
    assert np.isfinite(x0).all()
    np.testing.assert_allclose(x1, x0, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(e1, e0, rtol=1e-5, atol=1e-4)


def test_md_export_checkpoint_and_resume(tmp_path):
    """Exports, checkpoints and logs as base.py:799-1040 writes them; a run
    resumed from the checkpoint after the first export chunk writes the same
    second chunk, bit for bit, as the uninterrupted run (the noise is a
    function of the step counter, which the checkpoint restores)."""
    from mlcg_amd import nn
    from mlcg_amd.simulation import LangevinSimulation

    bonds = {(a, b): {"x_0": 3.8, "k": 5.0} for a in range(1, 6) for b in range(1, 6)}
    confs = _md_config(n_frames=3, n_beads=10, with_rep=False)
    for c in confs:
        for k in ("angles", "dihedrals"):
            c.neighbor_list.pop(k)

    def run(name, n_timesteps, capture, **kw):
        model = nn.SumOut(torch.nn.ModuleDict({"bonds": nn.GradientsOut(nn.HarmonicBonds(bonds))}))
        sim = LangevinSimulation(friction=1.0, dt=0.004, n_timesteps=n_timesteps,
                                 save_interval=5, export_interval=20, random_seed=11,
                                 capture=capture, save_energies=True, save_forces=True,
                                 filename=str(tmp_path / name), create_checkpoints=True,
                                 log_interval=20, **kw)
        sim.attach_model_and_configurations(model, [c.clone() for c in confs], L.beta_of(300.0))
        return sim, sim.simulate()

    _, last = run("a", 40, capture=False)
    a0 = np.load(tmp_path / "a_coords_0000.npy")
    a1 = np.load(tmp_path / "a_coords_0001.npy")
    assert a0.shape == (3, 4, 10, 3) and a1.shape == (3, 4, 10, 3)
    assert np.array_equal(last, a1)
    assert np.load(tmp_path / "a_potential_0001.npy").shape == (3, 4)
    assert np.load(tmp_path / "a_forces_0001.npy").shape == (3, 4, 10, 3)
    ck = torch.load(tmp_path / "a_checkpoint.pt", weights_only=True)
    assert ck["current_timestep"] == 2 and ck["export_interval"] == 20
    assert len(open(tmp_path / "a_log.txt").read().splitlines()) == 3  # header + 2 lines

    run("b", 20, capture=False)
    assert np.array_equal(np.load(tmp_path / "b_coords_0000.npy"), a0)
    sim, _ = run("b", 40, capture=False, read_checkpoint_file=True)
    assert sim.current_timestep == 1
    assert np.array_equal(np.load(tmp_path / "b_coords_0001.npy"), a1)
    assert np.array_equal(np.load(tmp_path / "b_potential_0001.npy"),
                          np.load(tmp_path / "a_potential_0001.npy"))


@pytest.mark.parametrize("capture", [False, True], ids=["eager", "captured"])
def test_md_overflow_between_checks_raises(capture):
    """A radius-graph capacity overflow on one intermediate step -- the
    chains are collapsed after step 4 and restored after step 5, so steps 5
    and 6 differ only in that step -- makes the run raise at its next check,
    although the last step's own graph flags are clean: every step's flags are
    ORed into one device flag inside the (captured) step."""
    from mlcg_amd import nn
    from mlcg_amd.simulation import LangevinSimulation

    confs = _md_config(n_frames=3, n_beads=60, with_rep=False)
    for c in confs:
        c.neighbor_list = {}

    def build():
        torch.manual_seed(0)
        rbf = nn.GaussianBasis(nn.CosineCutoff(0, 20.0), num_rbf=50)
        schnet = nn.StandardSchNet(rbf, nn.CosineCutoff(0, 20.0), [64], 128, 100, 128, 2,
                                   torch.nn.Tanh())
        return schnet, nn.SumOut(torch.nn.ModuleDict({"SchNet": nn.GradientsOut(schnet)}))

    for collapse in (False, True):
        schnet, model = build()
        sim = LangevinSimulation(friction=1.0, dt=0.004, n_timesteps=10, save_interval=10,
                                 random_seed=5, capture=capture, check_interval=1000,
                                 edge_capacity_factor=1.02)
        sim.attach_model_and_configurations(model, [c.clone() for c in confs], L.beta_of(300.0))
        saved = {}

        def hook(x, v, F, epot, step=[0]):
            step[0] += 1
            if not collapse:
                return
            if step[0] == 4:  # positions of step 5 collapse towards each frame's centre
                saved["x"], saved["v"] = x.clone(), v.clone()
                xf = x.view(3, 60, 3)
                xf.copy_(xf.mean(dim=1, keepdim=True) + 0.2 * (xf - xf.mean(dim=1, keepdim=True)))
            elif step[0] == 5:
                x.copy_(saved["x"])
                v.copy_(saved["v"])

        sim._hook, sim._hook_interval = hook, 1
        if not collapse:
            sim.simulate()
            e0 = schnet.last_graph.rowptr[-1].item()
            assert e0 < 0.9 * 3 * 60 * 59, "the test needs frames whose graph is not complete"
            continue
        with pytest.raises(RuntimeError, match="overflow"):
            sim.simulate()
        # the last step's own flags are clean: only the sticky flag saw it
        assert int(schnet.last_graph.flags.item()) == 0
