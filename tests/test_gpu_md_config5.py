"""Config 5's composite MD step -- SchNet (the config-2 architecture, rc 20 A)
plus harmonic bonds and angles, 3-term Fourier dihedrals and the (sigma/r)^6
repulsion, integrated by BAOAB with the radius graph rebuilt every step --
against the CPU oracles chained together:
  forces  oracle/schnet_ref.py (fp64 SchNet, oracle radius graph at rc 20)
          + oracle/priors_ref.py (the four priors with the config-5 constants)
  step    oracle/langevin_ref.py (LangevinSimulation.timestep,
          mlcg/simulation/langevin.py:100-144), fed the normals the HIP step
          draws (ops.philox_normals at the same step counter).
Every step of the HIP run (eager and captured) is checked from the state the
HIP run itself reached, so the oracle never drifts along a chaotic trajectory:
the forces and potential energies at the step's positions, and the positions
and velocities of the next step.

Tolerances, per element (tests.helpers.check): forces rtol 1e-5 (the
energy/force bar of north_star); positions rtol 1e-6 (one fp32 rounding of a
coordinate of up to ~40 A on a displacement of ~0.02 A per step); velocities
rtol 1e-5 (they carry the force error through 0.5 dt F / m).
"""

import numpy as np
import pytest
import torch

from oracle import langevin_ref as L
from oracle import priors_ref as P
from oracle import radius as oracle_radius
from oracle import schnet_ref as R
from tests.helpers import check

pytestmark = pytest.mark.gpu

N_BEADS = 268
SEED = 20265


def _model():
    from mlcg_amd import nn, synthetic

    torch.manual_seed(synthetic.seed_for(5))
    rbf = nn.GaussianBasis(nn.CosineCutoff(0.0, 20.0), num_rbf=50)
    schnet = nn.StandardSchNet(rbf, nn.CosineCutoff(0.0, 20.0), [64], 128, 100, 128, 3,
                               torch.nn.Tanh())
    models = {"SchNet": nn.GradientsOut(schnet)}
    for k, v in synthetic.config5_prior_models().items():
        models[k] = nn.GradientsOut(v)
    return schnet, nn.SumOut(torch.nn.ModuleDict(models))


def _oracle_force_fn(schnet, n_frames, types, double_graph=False):
    """Total force of the composite model at given positions, in fp64 (the
    radius graph searched in float32 as the float32 model does, or in double
    for a model moved to double)."""
    import math

    from mlcg_amd import synthetic

    c = synthetic.CONFIG5_PRIORS
    sd = {k: v.detach().double().cpu() for k, v in schnet.state_dict().items()}
    cfg = R.SchNetConfig(num_rbf=50, rbf_lo=0.0, rbf_hi=20.0, rbf_cut="cosine",
                         conv_cut="cosine", conv_lo=0.0, conv_hi=20.0, act="tanh",
                         num_blocks=3)
    topo = P.chain_topology(n_frames, N_BEADS, min_sep=c["repulsion"]["min_separation"])
    batch = torch.arange(n_frames).repeat_interleave(N_BEADS)

    def full(M, v):
        return torch.full((M,), float(v), dtype=torch.float64)

    params = {}
    M = topo["bonds"][0].shape[1]
    params["bonds"] = {"x0": full(M, c["bonds"]["x_0"]), "k": full(M, c["bonds"]["k"])}
    M = topo["angles"][0].shape[1]
    params["angles"] = {"x0": full(M, math.cos(math.radians(c["angles"]["theta_0_deg"]))),
                        "k": full(M, c["angles"]["k"])}
    M = topo["dihedrals"][0].shape[1]
    d = c["dihedrals"]
    params["dihedrals"] = {"v_0": full(M, d["v_0"]),
                           "k1s": torch.tensor(d["k1s"], dtype=torch.float64).repeat(M, 1),
                           "k2s": torch.tensor(d["k2s"], dtype=torch.float64).repeat(M, 1)}
    M = topo["repulsion"][0].shape[1]
    params["repulsion"] = {"sigma": full(M, c["repulsion"]["sigma"])}

    def forces(x64):
        xg = x64.numpy() if double_graph else x64.float().numpy()
        ei, ovf = oracle_radius.radius_graph(xg, 20.0, batch.numpy(), False, 1000)
        assert ovf == 0
        E, F = R.schnet_energy_forces(sd, cfg, x64, types, batch, torch.from_numpy(ei),
                                      n_frames)
        for kind, (mapping, mb) in topo.items():
            Ek, Fk = P.prior_energy_forces(kind, x64, mapping, mb, n_frames, params[kind])
            E = E + Ek
            F = F + Fk
        return E.detach(), F.detach()

    return forces


@pytest.mark.parametrize("capture", [False, True], ids=["eager", "captured"])
def test_config5_composite_steps_vs_oracle(capture):
    from mlcg_amd import ops, synthetic
    from mlcg_amd.simulation import LangevinSimulation

    n_frames, n_steps = 4, 6
    print(f"config-5 composite step, {n_frames} x {N_BEADS} beads, capture={capture}",
          flush=True)
    c = synthetic.CONFIG5_PRIORS
    schnet, model = _model()
    confs = synthetic.config5_configurations(n_frames=n_frames, n_beads=N_BEADS)
    beta = L.beta_of(c["temperature_K"])
    sim = LangevinSimulation(friction=c["friction_per_ps"], dt=c["dt_ps"],
                             n_timesteps=n_steps, save_interval=1, random_seed=SEED,
                             capture=capture)
    sim.attach_model_and_configurations(model, confs, beta)
    states = []
    sim._hook = lambda x, v, F, e: states.append(
        tuple(t.detach().double().cpu().clone() for t in (x, v, F, e)))
    sim._hook_interval = 1
    sim.simulate()
    assert len(states) == n_steps
    types = torch.cat([d.atom_types for d in confs])
    forces = _oracle_force_fn(schnet, n_frames, types)
    m = sim.initial_data.masses.double().cpu()
    bmr = torch.sqrt(1.0 / (beta * m))
    vscale, noisescale = L.constants(c["dt_ps"], c["friction_per_ps"])
    N = m.numel()
    oracle = [forces(s[0]) for s in states]  # (E, F) at every state's positions
    for k in range(n_steps):
        _, _, F, epot = states[k]
        check(F, oracle[k][1], 1e-5, f"step {k} forces")
        check(epot, oracle[k][0], 1e-5, f"step {k} potential energies")
    for k in range(n_steps - 1):
        x, v, _, _ = states[k]
        xn, vn, _, _ = states[k + 1]
        # the next step from this state, with the normals the kernel drew at
        # step counter k + 1; the closing half-kick takes the force at the
        # positions the HIP step reached (with stiff bonds, 2k = 200
        # kcal/mol/A^2, a position difference of one fp32 rounding would
        # already move that force by ~1e-3)
        xi = ops.philox_normals(SEED, k + 1, N, "cuda").double().cpu()
        x1, v1 = L.baoa(x, v, oracle[k][1], m, bmr, c["dt_ps"], vscale, noisescale, xi)
        v1 = L.b(v1, oracle[k + 1][1], m, c["dt_ps"])
        check(xn, x1, 1e-6, f"step {k + 1} positions")
        check(vn, v1, 1e-5, f"step {k + 1} velocities")


def test_config5_full_size_captured_run():
    """The full config-5 system (100 x 268 beads): a captured run stays
    finite, never overflows its radius-graph capacity (the simulation raises
    otherwise), and its steps after the capture equal those of the eager run.
    Three of its frames (0, 57, 99: each frame is an independent system) are
    checked against the chained fp64 oracles as in the 4-frame test:
    forces and potential energies at every replayed step, and the positions
    and velocities of each replayed step from the state before it."""
    from mlcg_amd import ops, synthetic
    from mlcg_amd.simulation import LangevinSimulation

    c = synthetic.CONFIG5_PRIORS
    trajs = []
    states = []
    schnet = None
    for capture in (False, True):
        print(f"config-5 full size, capture={capture}", flush=True)
        schnet, model = _model()
        sim = LangevinSimulation(friction=c["friction_per_ps"], dt=c["dt_ps"], n_timesteps=6,
                                 save_interval=1, random_seed=SEED, capture=capture,
                                 save_energies=True, check_interval=1)
        confs = synthetic.config5_configurations()
        sim.attach_model_and_configurations(model, confs, L.beta_of(c["temperature_K"]))
        if capture:
            sim._hook = lambda x, v, F, e: states.append(
                tuple(t.detach().double().cpu().clone() for t in (x, v, F, e)))
            sim._hook_interval = 1
        x = sim.simulate()
        assert np.isfinite(x).all() and np.isfinite(sim.simulated_potential).all()
        trajs.append((x, sim.simulated_potential))
    (xe, ee), (xc, ec) = trajs
    assert xe.shape == (100, 6, N_BEADS, 3)
    # the capture happens at step 3; steps 3..6 are replays
    np.testing.assert_allclose(xc[:, 2:], xe[:, 2:], rtol=1e-6, atol=1e-5)
    np.testing.assert_allclose(ec[:, 2:], ee[:, 2:], rtol=1e-5, atol=1e-4)

    assert len(states) == 6
    beta = L.beta_of(c["temperature_K"])
    m_all = sim.initial_data.masses.double().cpu()
    vscale, noisescale = L.constants(c["dt_ps"], c["friction_per_ps"])
    # the three frames are checked together, as one system of three frames
    # (the element-wise bound's absolute term scales with that system's
    # largest force, as in the 4-frame test above)
    frames = (0, 57, 99)
    idx = torch.cat([torch.arange(f * N_BEADS, (f + 1) * N_BEADS) for f in frames])
    types_all = torch.cat([d.atom_types for d in confs])
    forces = _oracle_force_fn(schnet, len(frames), types_all[idx])
    m = m_all[idx]
    bmr = torch.sqrt(1.0 / (beta * m))
    oracle = {k: forces(states[k][0][idx]) for k in range(1, 6)}
    for k in range(2, 6):  # steps 3..6: graph replays
        _, _, F, epot = states[k]
        check(F[idx], oracle[k][1], 1e-5, f"frames {frames} step {k} forces")
        check(epot[list(frames)], oracle[k][0], 1e-5, f"frames {frames} step {k} energies")
        x, v = (t[idx] for t in states[k - 1][:2])
        xi = ops.philox_normals(SEED, k, m_all.numel(), "cuda").double().cpu()[idx]
        x1, v1 = L.baoa(x, v, oracle[k - 1][1], m, bmr, c["dt_ps"], vscale, noisescale, xi)
        v1 = L.b(v1, oracle[k][1], m, c["dt_ps"])
        check(states[k][0][idx], x1, 1e-6, f"frames {frames} step {k} positions")
        check(states[k][1][idx], v1, 1e-5, f"frames {frames} step {k} velocities")


def test_double_precision_composite_steps_vs_oracle():
    """LangevinSimulation(dtype="double") (the reference moves the model to
    double, base.py:162,271): SchNet module by module in float64 (HIP float64
    gather and per-frame sums, torch linears), the four priors and BAOAB on
    their float64 kernels, radius graph in double.  Against the fp64 oracles
    chained as above (oracle radius graph searched in double) at rtol 1e-9 on
    forces, energies, positions and velocities -- four orders tighter than a
    float32 computation could meet."""
    from mlcg_amd import ops, synthetic
    from mlcg_amd.simulation import LangevinSimulation

    n_frames, n_steps = 2, 4
    c = synthetic.CONFIG5_PRIORS
    schnet, model = _model()
    confs = synthetic.config5_configurations(n_frames=n_frames, n_beads=N_BEADS)
    beta = L.beta_of(c["temperature_K"])
    sim = LangevinSimulation(friction=c["friction_per_ps"], dt=c["dt_ps"],
                             n_timesteps=n_steps, save_interval=1, random_seed=SEED,
                             dtype="double")
    sim.attach_model_and_configurations(model, confs, beta)
    assert all(p.dtype == torch.float64 for p in model.parameters())
    assert schnet.fused_spec() is None
    # the priors' tables hold float32 roundings of the constants until refilled
    # in double (the oracle uses the exact constants)
    synthetic.fill_config5_prior_constants(
        {k: model.models[k].model for k in ("bonds", "angles", "dihedrals", "repulsion")})
    states = []
    sim._hook = lambda x, v, F, e: states.append(
        tuple(t.detach().cpu().clone() for t in (x, v, F, e)))
    sim._hook_interval = 1
    sim.simulate()
    assert len(states) == n_steps and all(t.dtype == torch.float64 for t in states[0])
    types = torch.cat([d.atom_types for d in confs])
    forces = _oracle_force_fn(schnet, n_frames, types, double_graph=True)
    m = sim.initial_data.masses.double().cpu()
    bmr = torch.sqrt(1.0 / (beta * m))
    vscale, noisescale = L.constants(c["dt_ps"], c["friction_per_ps"])
    N = m.numel()
    oracle = [forces(s[0]) for s in states]
    for k in range(n_steps):
        _, _, F, epot = states[k]
        check(F, oracle[k][1], 1e-9, f"double step {k} forces")
        check(epot, oracle[k][0], 1e-9, f"double step {k} potential energies")
    for k in range(n_steps - 1):
        x, v, _, _ = states[k]
        xn, vn, _, _ = states[k + 1]
        xi = ops.philox_normals(SEED, k + 1, N, "cuda").double().cpu()
        x1, v1 = L.baoa(x, v, oracle[k][1], m, bmr, c["dt_ps"], vscale, noisescale, xi)
        v1 = L.b(v1, oracle[k + 1][1], m, c["dt_ps"])
        check(xn, x1, 1e-9, f"double step {k + 1} positions")
        check(vn, v1, 1e-9, f"double step {k + 1} velocities")


def test_compiled_simulation_matches_eager():
    """LangevinSimulation(compile=True): the model goes through
    torch.compile(dynamic=True) with the default (inductor) backend at the
    start of simulate(), as the reference's simulation does (base.py:447-489);
    its energies, forces and trajectory equal the eager run's within the
    reference's own compiled-vs-eager bar (rtol = atol = 1e-5,
    tests/unit/simulation/test_compilation.py:264-269)."""
    from mlcg_amd import synthetic
    from mlcg_amd.simulation import LangevinSimulation

    n_frames, n_steps = 4, 4
    c = synthetic.CONFIG5_PRIORS
    runs = []
    for compile_flag in (False, True):
        print(f"config-5 composite step, {n_frames} x {N_BEADS} beads, compile={compile_flag}",
              flush=True)
        _, model = _model()
        sim = LangevinSimulation(friction=c["friction_per_ps"], dt=c["dt_ps"],
                                 n_timesteps=n_steps, save_interval=1, random_seed=SEED,
                                 save_energies=True, save_forces=True, compile=compile_flag)
        sim.attach_model_and_configurations(
            model, synthetic.config5_configurations(n_frames=n_frames, n_beads=N_BEADS),
            L.beta_of(c["temperature_K"]))
        import warnings

        import torch._dynamo.utils

        torch._dynamo.utils.counters.clear()
        with warnings.catch_warnings(record=True) as caught:
            warnings.simplefilter("always")
            x = sim.simulate()
        # compiled without the suppress_errors fallback
        assert not any("torch.compile failed" in str(w.message) for w in caught)
        assert isinstance(sim.model, torch._dynamo.eval_frame.OptimizedModule) == compile_flag
        breaks = dict(torch._dynamo.utils.counters["graph_break"])
        print(f"  graph breaks: {sum(breaks.values())} ({len(breaks)} reasons)", flush=True)
        for reason in list(breaks)[:6]:
            print("   ", " | ".join(reason.splitlines()[:4])[:600], flush=True)
        # the HIP passes are custom operators: the model compiles as one graph
        assert not breaks
        runs.append((x, sim.simulated_potential, sim.simulated_forces))
    for a, b, what in zip(runs[1], runs[0], ("positions", "energies", "forces")):
        np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-5, err_msg=what)


def test_compiled_model_fullgraph_bit_identical():
    """The config-5 model (SumOut of GradientsOut around SchNet and the four
    priors) compiles as one graph: torch.compile(fullgraph=True, dynamic=True)
    traces the HIP passes through the fake kernels of mlcg::direct_energy_forces
    and mlcg::sum_arrays, and the compiled call runs the same kernels, so its
    energies and forces equal the eager ones bit for bit (inductor backend)."""
    import torch._dynamo

    from mlcg_amd import synthetic
    from mlcg_amd.data._keys import ENERGY_KEY, FORCE_KEY
    from mlcg_amd.simulation import LangevinSimulation

    c = synthetic.CONFIG5_PRIORS
    _, model = _model()
    sim = LangevinSimulation(friction=c["friction_per_ps"], dt=c["dt_ps"], n_timesteps=2,
                             save_interval=1, random_seed=SEED)
    sim.attach_model_and_configurations(
        model, synthetic.config5_configurations(n_frames=4, n_beads=N_BEADS),
        L.beta_of(c["temperature_K"]))
    e_ref, f_ref = sim.calculate_potential_and_forces(sim.initial_data.clone())
    torch._dynamo.reset()
    compiled = torch.compile(sim.model, fullgraph=True, dynamic=True)
    for rep in range(2):
        print(f"compiled call {rep}", flush=True)
        out = compiled(sim.initial_data.clone())
        torch.cuda.synchronize()
        assert torch.equal(out.out[ENERGY_KEY], e_ref)
        assert torch.equal(out.out[FORCE_KEY], f_ref)
