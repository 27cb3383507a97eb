"""Host-side logic that needs no GPU: the C-ABI library loads and exports
every entry point declared in include/mlcg_hip.h, the Python wrappers refuse
CPU tensors loudly, the module API keeps the reference's constructor
behaviour and state_dict layout, and AtomicData collation follows the
reference's increment rules."""

import os
import re
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    names = []
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[\w\*\s]+?\b(mlcg_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    from mlcg_amd import _lib

    lib = _lib.load()
    declared = _declared_symbols()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), name
    # and the Python binding binds exactly the declared set
    assert sorted(_lib.exported_symbols()) == declared
    assert "gfx950" in _lib.version()


def test_library_symbols_in_dynamic_table():
    so = os.path.join(ROOT, "mlcg_amd", "libmlcg_hip.so")
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (mlcg_\w+)", out))
    assert set(_declared_symbols()) <= exported


def test_wrappers_refuse_cpu_tensors():
    from mlcg_amd import ops

    pos = torch.zeros(4, 3)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.radius_graph(pos, 1.0)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.frame_ptr_from_batch(torch.zeros(4, dtype=torch.long), 1)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.segment_sum(torch.zeros(4), torch.tensor([0, 4]))


def test_missing_library_raises(monkeypatch, tmp_path):
    from mlcg_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    assert not _lib.available()
    with pytest.raises(RuntimeError, match="not found"):
        _lib.call("mlcg_version")


def test_model_forward_refuses_cpu():
    from mlcg_amd import nn, synthetic

    m = _config2_model(nn)
    data = synthetic.config2(n_frames=2).to_torch("cpu")
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        nn.GradientsOut(m)(data)


def _config2_model(nn, act=None):
    act = act or torch.nn.Tanh()
    rbf = nn.GaussianBasis(nn.CosineCutoff(0, 20), num_rbf=50)
    return nn.StandardSchNet(rbf, nn.CosineCutoff(0, 20), [64], 128, 100, 128, 3, act)


def test_state_dict_contract():
    """Keys and shapes of StandardSchNet (config 2) follow the reference's
    module tree (schnet.py:86-105,219-221,295-298, mlp.py:49)."""
    from mlcg_amd import nn

    sd = _config2_model(nn).state_dict()
    want = {"embedding_layer.weight": (100, 128), "rbf_layer.offset": (50,),
            "rbf_layer.coeff": (), "output_network.layers.0.weight": (64, 128),
            "output_network.layers.0.bias": (64,), "output_network.layers.2.weight": (1, 64)}
    for b in range(3):
        p = f"interaction_blocks.{b}"
        want.update({f"{p}.conv.lin1.weight": (128, 128), f"{p}.conv.lin2.weight": (128, 128),
                     f"{p}.conv.lin2.bias": (128,),
                     f"{p}.conv.filter_network.layers.0.weight": (128, 50),
                     f"{p}.conv.filter_network.layers.0.bias": (128,),
                     f"{p}.conv.filter_network.layers.2.weight": (128, 128),
                     f"{p}.lin.weight": (128, 128), f"{p}.lin.bias": (128,)})
    assert {k: tuple(v.shape) for k, v in sd.items()} == want
    m = _config2_model(nn)
    assert sum(p.numel() for p in m.parameters()) == 238_080
    g = nn.GradientsOut(m)
    assert all(k.startswith("model.") for k in g.state_dict())


def test_standard_schnet_checks():
    from mlcg_amd import nn

    rbf = nn.GaussianBasis(nn.CosineCutoff(0, 20), num_rbf=50)
    with pytest.raises(ValueError):
        nn.StandardSchNet(rbf, nn.CosineCutoff(0, 20), [64], num_interactions=0)
    with pytest.warns(UserWarning):
        nn.StandardSchNet(rbf, nn.CosineCutoff(0, 15), [64], num_interactions=1)
    with pytest.raises(NotImplementedError):
        nn.SchNet(torch.nn.Embedding(10, 128), [], rbf, nn.MLP([128, 1]),
                  self_interaction=True)


@pytest.mark.parametrize("cls", ["IdentityCutoff", "CosineCutoff"])
def test_cutoff_bounds_raise(cls):
    from mlcg_amd import nn

    with pytest.raises(ValueError):
        getattr(nn, cls)(cutoff_lower=10, cutoff_upper=0)


@pytest.mark.parametrize("basis,default_cutoff", [("GaussianBasis", "IdentityCutoff"),
                                                   ("ExpNormalBasis", "CosineCutoff")])
def test_basis_float_cutoff_defaults(basis, default_cutoff):
    """tests/unit/nn/radial_basis/test_radial_basis.py:12-44."""
    from mlcg_amd import nn

    b = getattr(nn, basis)(cutoff=10)
    assert isinstance(b.cutoff, getattr(nn, default_cutoff))
    assert b.cutoff.cutoff_lower == 0 and b.cutoff.cutoff_upper == 10
    with pytest.raises(ValueError):
        getattr(nn, basis)(cutoff=nn.IdentityCutoff(cutoff_lower=10, cutoff_upper=0))


def test_expnormal_module_matches_oracle():
    """ExpNormalBasis: parameter/buffer registration and state_dict keys
    (exp_normal.py:72-78), initial values and forward against the oracle."""
    from mlcg_amd import nn
    from oracle import schnet_ref as R

    b = nn.ExpNormalBasis(nn.CosineCutoff(0.0, 12.0), num_rbf=16)
    assert b.trainable and b.alpha == pytest.approx(5.0 / 12.0)
    assert {k for k, _ in b.named_parameters()} == {"means", "betas"}
    fixed = nn.ExpNormalBasis(12.0, num_rbf=16, trainable=False)
    assert not list(fixed.parameters()) and set(fixed.state_dict()) == {"means", "betas"}
    means, betas = R.expnormal_params(0.0, 12.0, 16)
    assert torch.equal(b.means.data, means) and torch.equal(b.betas.data, betas)
    d = torch.linspace(0.0, 13.0, 40)
    ref = R.expnormal_rbf(d.double(), means.double(), betas.double(), 5.0 / 12.0, 0.0,
                          R.Cutoff("cosine", 0.0, 12.0))
    assert torch.allclose(b(d).double(), ref, rtol=1e-5, atol=1e-7)
    with torch.no_grad():
        b.means.mul_(2.0)
    b.reset_parameters()
    assert torch.equal(b.means.data, means)


@pytest.mark.parametrize("basis,key", [("GaussianBasis", "offset"), ("ExpNormalBasis", "means")])
@pytest.mark.parametrize("trainable", [False, True])
def test_pruned_basis(basis, key, trainable):
    """build_pruned_from_mask (gaussian.py:104-153, exp_normal.py:126-178)."""
    from mlcg_amd import nn

    mask = torch.tensor([True, False, True, True, False, False, True, False])
    full = getattr(nn, basis)(nn.CosineCutoff(0.0, 8.0), num_rbf=8, trainable=trainable)
    pr = getattr(nn, basis).build_pruned_from_mask(nn.CosineCutoff(0.0, 8.0), mask,
                                                    num_rbf=8, trainable=trainable)
    assert torch.equal(getattr(pr, key).data, getattr(full, key).data[mask])
    assert pr.num_rbf == 8  # the reference keeps the unpruned count
    assert (key in dict(pr.named_parameters())) == trainable
    d = torch.linspace(0.1, 7.9, 9)
    assert torch.allclose(pr(d), full(d)[:, mask])
    with pytest.raises(ValueError):
        getattr(nn, basis).build_pruned_from_mask(8.0, mask[:5], num_rbf=8)


def test_fused_spec_recognises_config2():
    from mlcg_amd import nn

    m = _config2_model(nn)
    spec = m.fused_spec()
    assert spec is not None and spec.num_blocks == 3 and spec.filt.num_rbf == 50
    m2 = _config2_model(nn, act=torch.nn.ReLU())
    assert m2.fused_spec() is None  # no kernel for ReLU: module-by-module path


def test_cfconv_aggregations():
    """CFConv takes PyG's "add" / "sum" (fused path) and "mean" (module by
    module: the HIP gather divided by the in-degree); other aggregations
    raise at construction."""
    from mlcg_amd import nn

    rbf = nn.GaussianBasis(nn.CosineCutoff(0.0, 20.0), num_rbf=50)
    for aggr, fused in (("add", True), ("sum", True), ("mean", False)):
        m = nn.StandardSchNet(rbf, nn.CosineCutoff(0.0, 20.0), [64], num_interactions=2,
                              embedding_size=21, aggr=aggr)
        assert all(b.conv.aggr == aggr for b in m.interaction_blocks)
        assert (m.fused_spec() is not None) == fused, aggr
    with pytest.raises(NotImplementedError, match="aggr='max'"):
        nn.StandardSchNet(rbf, nn.CosineCutoff(0.0, 20.0), [64], aggr="max")


@pytest.mark.parametrize("trainable", [False, True])
def test_fused_spec_basis_kinds(trainable):
    """Both bases, trainable or fixed, have a fused spec; its basis tensors
    alias the module's own float32 parameters."""
    from mlcg_amd import nn, ops

    for cls, kind in ((nn.GaussianBasis, ops.BASIS_GAUSSIAN),
                      (nn.ExpNormalBasis, ops.BASIS_EXPNORMAL)):
        rbf = cls(nn.CosineCutoff(0, 20), num_rbf=50, trainable=trainable)
        m = nn.StandardSchNet(rbf, nn.CosineCutoff(0, 20), [64], 128, 100, 128, 2,
                              torch.nn.Tanh())
        spec = m.fused_spec()
        assert spec is not None and spec.filt.basis == kind
        assert spec.basis_trainable == trainable
        c = rbf.offset if cls is nn.GaussianBasis else rbf.means
        assert spec.filt.centers.data_ptr() == c.data_ptr()
        P = m.fused_params()
        assert len(P.flat()) == 1 + 8 * 2 + 3 + (2 if trainable else 0)
        if kind == ops.BASIS_EXPNORMAL:
            assert spec.filt.alpha == pytest.approx(0.25)


def test_collate_increments_index_keys():
    from mlcg_amd.data import AtomicData
    from mlcg_amd.data.atomic_data import collate

    frames = []
    for n in (3, 4):
        nl = {"bonds": {"index_mapping": torch.tensor([[0, 1], [1, 2]]), "order": 2}}
        frames.append(AtomicData.from_points(torch.zeros(n, 3), torch.arange(n),
                                             neighborlist=nl))
    b = collate(frames)
    assert b.batch.tolist() == [0, 0, 0, 1, 1, 1, 1]
    assert b.neighbor_list["bonds"]["index_mapping"].tolist() == [[0, 1, 3, 4], [1, 2, 4, 5]]
    assert b.neighbor_list["bonds"]["mapping_batch"].tolist() == [0, 0, 1, 1]
    assert b.n_atoms.tolist() == [3, 4]


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_bench_algorithmic_work_formulas():
    """Per-launch algorithmic figures used by bench.py's roofline."""
    sys.path.insert(0, ROOT)
    import bench

    E, P, N, B = 1000, 500, 100, 4
    bound, flops, _ = bench.algorithmic_work("mlcg_filter_fwd", E, P, N, B)
    assert bound == "mfma" and flops == 2 * 2 * (50 * 128 + 128 * 128) * P
    bound, byts, _ = bench.algorithmic_work("mlcg_cfconv_gather", E, P, N, B)
    assert bound == "hbm" and byts == 4 * 128 * P + 4 * E + 4 * (N + 1) + 8 * 128 * N


def test_exclusion_pair_to_ptr_host_abi():
    """mlcg_exclusion_pair_to_ptr is a host function of the C ABI (the
    reference converts on the host too, exclusion_pairs.cpp:7-62): checked
    against the oracle's restatement, including duplicates, centres past the
    last node, an empty list and the negative-centre error."""
    import numpy as np

    from mlcg_amd import ops
    from oracle import radius as oracle_radius

    rng = np.random.default_rng(2)
    for n, m in [(1, 3), (17, 0), (50, 400), (200, 5000)]:
        x = rng.integers(-3, n + 3, m)
        y = rng.integers(0, n + 2, m)
        exc = np.stack([x, y]).astype(np.int64)
        xs, yp = ops.exclusion_pair_to_ptr(torch.from_numpy(exc), n)
        want_xs, want_yp = oracle_radius.exclusion_pair_to_ptr(exc, n)
        assert xs.dtype == torch.int64 and yp.dtype == torch.int64
        assert np.array_equal(xs.numpy(), want_xs)
        assert np.array_equal(yp.numpy(), want_yp)
    with pytest.raises(RuntimeError):
        ops.exclusion_pair_to_ptr(torch.tensor([[0, 1], [-1, 0]]), 3)
    xs, yp = ops.exclusion_pair_to_ptr(torch.tensor([[0, 1], [-1, 0]]), 0)
    assert yp.tolist() == [0] and xs.tolist() == [0, 1]
    with pytest.raises(RuntimeError):
        ops.exclusion_pair_to_ptr(torch.tensor([[0, 1], [1, 0]], dtype=torch.int32), 3)


def test_langevin_export_options_are_checked():
    from mlcg_amd.simulation import LangevinSimulation

    with pytest.raises(ValueError, match="filename"):
        LangevinSimulation(n_timesteps=100, save_interval=10, export_interval=50)
    with pytest.raises(ValueError, match="filename"):
        LangevinSimulation(n_timesteps=100, save_interval=10, create_checkpoints=True)
    with pytest.raises(ValueError, match="multiple of save_interval"):
        LangevinSimulation(n_timesteps=100, save_interval=10, export_interval=25, filename="x")
    with pytest.raises(ValueError, match="multiple of export_interval"):
        LangevinSimulation(n_timesteps=100, save_interval=10, export_interval=30, filename="x")
    with pytest.raises(ValueError, match="log_type"):
        LangevinSimulation(n_timesteps=100, save_interval=10, log_interval=10, log_type="x")
    sim = LangevinSimulation(n_timesteps=100, save_interval=10, log_interval=10,
                             log_type="print", device="cpu")
    assert sim.export_interval == 100 and sim.filename is None


def test_reference_operators_registered_with_fake_kernels():
    """Importing the package registers the reference's operator names
    (radius.cu:313-314, exclusion_pairs.cpp:64-65) as torch.library custom
    ops; their fake kernels give torch.compile the output shapes (an unbacked
    edge count for the radius graph) without running anything."""
    import mlcg_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.fx.experimental.symbolic_shapes import ShapeEnv

    assert torch.ops.mlcg.radius_cuda is not None
    assert torch.ops.mlcg.exclusion_pair_to_ptr is not None
    with FakeTensorMode(shape_env=ShapeEnv()):
        x = torch.empty(10, 3, dtype=torch.float64)
        ei, d = torch.ops.mlcg.radius_cuda(x, None, 1.0, 8, True)
        assert ei.dim() == 2 and ei.shape[0] == 2 and ei.dtype == torch.int64
        assert d.dtype == torch.float64 and d.shape[0] == ei.shape[1]
        xs, ptr = torch.ops.mlcg.exclusion_pair_to_ptr(torch.empty(2, 5, dtype=torch.int64), 7)
        assert tuple(xs.shape) == (5,) and tuple(ptr.shape) == (8,)


def test_model_operators_fake_kernels_and_registry():
    """mlcg::direct_energy_forces and mlcg::sum_arrays (the fused passes as
    torch.compile sees them): the fake kernels give energies [n_frames] and
    forces [N, 3] from the batch's n_atoms, and the sum's shape; GradientsOut
    registers the model it wraps under id(model), again for a deep copy (which
    holds a new model object), and an unregistered id is refused."""
    import copy

    import mlcg_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.fx.experimental.symbolic_shapes import ShapeEnv

    from mlcg_amd import library, nn

    with FakeTensorMode(shape_env=ShapeEnv()):
        pos = torch.empty(12, 3)
        types = torch.empty(12, dtype=torch.int64)
        batch = torch.empty(12, dtype=torch.int64)
        n_atoms = torch.empty(4, dtype=torch.int64)
        E, F = torch.ops.mlcg.direct_energy_forces(pos, types, batch, n_atoms, None, None, 1)
        assert tuple(E.shape) == (4,) and tuple(F.shape) == (12, 3)
        assert E.dtype == F.dtype == torch.float32
        S = torch.ops.mlcg.sum_arrays([pos, pos, pos])
        assert tuple(S.shape) == (12, 3)

    prior = nn.HarmonicBonds({(1, 2): {"x_0": 1.0, "k": 2.0}})
    g = nn.GradientsOut(prior)
    assert library._DIRECT_MODELS[id(prior)] is prior
    g2 = copy.deepcopy(g)
    assert g2.model is not prior and library._DIRECT_MODELS[id(g2.model)] is g2.model
    unused = max(library._DIRECT_MODELS.keys()) + 8
    with pytest.raises(RuntimeError, match="no model registered"):
        torch.ops.mlcg.direct_energy_forces(torch.zeros(2, 3), torch.zeros(2, dtype=torch.int64),
                                            torch.zeros(2, dtype=torch.int64),
                                            torch.ones(1, dtype=torch.int64), None, None, unused)


def test_mfma_probe_flop_counts():
    """The MFMA-loop probe's FLOP count per wave iteration (host-side, no
    GPU): 8 chains of 2·M·N·K for each shape, -1 for an unknown kind."""
    from mlcg_amd import _lib

    lib = _lib.load()
    shapes = {0: (16, 16, 32), 1: (16, 16, 16), 2: (16, 16, 4), 3: (16, 16, 32), 4: (32, 32, 16)}
    for kind, (m, n, k) in shapes.items():
        assert lib.mlcg_mfma_loop_flops_per_wave_iter(kind) == 8 * 2 * m * n * k
    assert lib.mlcg_mfma_loop_flops_per_wave_iter(5) == -1


def test_radius_flag_bookkeeping():
    """Every bit of the radius graph's flag word is named, and a look-back
    timeout (bit 8) discards the cached look-back workspaces so that the next
    call starts from a zero-filled one (other bits keep them)."""
    from mlcg_amd import ops

    assert ops.radius_flags_message(0) == "none"
    msg = ops.radius_flags_message(1 | 2 | 4 | 8 | 16, capacity=100)
    for part in ("max_num_neighbors", "capacity 100", "not symmetric", "look-back", "2^31"):
        assert part in msg, (part, msg)
    ops._RADIUS_WS[(0, 1)] = "workspace"
    ops.radius_flags_read(1 | 2 | 4 | 16)
    assert (0, 1) in ops._RADIUS_WS
    ops.radius_flags_read(8)
    assert not ops._RADIUS_WS


def test_langevin_dtype_options():
    """LangevinSimulation takes dtype "single" and "double" (base.py:162); a
    double run is not captured; other dtypes raise."""
    from mlcg_amd.simulation import LangevinSimulation

    assert LangevinSimulation(dtype="single").dtype == torch.float32
    assert LangevinSimulation(dtype="double").dtype == torch.float64
    with pytest.raises(ValueError, match="capture"):
        LangevinSimulation(dtype="double", capture=True)
    with pytest.raises(ValueError, match="dtype"):
        LangevinSimulation(dtype="half")


def test_simulation_compile_model_options(monkeypatch):
    """compile_model follows the reference's control flow (base.py:447-489):
    one structure stays eager with a warning unless force_compile; otherwise
    torch.compile(model, dynamic=True, mode=compile_mode) and one checked
    call; when the compiled call raises, dynamo's suppress_errors is set and
    the model compiled again.  torch.compile is replaced by a recorder here
    (the real compile of the HIP model runs in the GPU tests)."""
    import warnings

    import torch._dynamo

    from mlcg_amd.data._keys import ENERGY_KEY, FORCE_KEY
    from mlcg_amd.simulation import LangevinSimulation

    class Toy(torch.nn.Module):
        def forward(self, data):
            data.out = {ENERGY_KEY: data.pos.sum().reshape(1), FORCE_KEY: -data.pos}
            return data

    class Data:
        def __init__(self, n_frames):
            self.pos = torch.ones(2 * n_frames, 3)
            self.batch = torch.arange(n_frames).repeat_interleave(2)
            self.out = {}

    calls = []

    def fake_compile(model, dynamic=None, mode=None):
        calls.append((dynamic, mode))
        if len(calls) == 1 and failing[0]:
            class Broken(torch.nn.Module):
                def __init__(self):
                    super().__init__()
                    self._orig_mod = model

                def forward(self, data):
                    raise RuntimeError("unsupported")
            return Broken()
        return model

    monkeypatch.setattr(torch, "compile", fake_compile)
    monkeypatch.setattr(torch._dynamo.config, "suppress_errors", False)
    failing = [False]
    with pytest.raises(ValueError):
        LangevinSimulation(device="cpu", compile=True, capture=True)
    for mode in ("reduce-overhead", "max-autotune"):
        with pytest.raises(ValueError, match="capture=True"):
            LangevinSimulation(device="cpu", compile=True, compile_mode=mode)
    sim = LangevinSimulation(device="cpu", compile=True, compile_mode="max-autotune-no-cudagraphs")
    sim.model = Toy()
    with pytest.warns(UserWarning, match="more than one structure"):
        sim.compile_model(Data(1))
    assert calls == []
    sim.compile_model(Data(2))
    assert calls == [(True, "max-autotune-no-cudagraphs")]
    sim = LangevinSimulation(device="cpu", compile=True, force_compile=True)
    sim.model = Toy()
    calls.clear()
    with pytest.warns(UserWarning, match="one structure"):
        sim.compile_model(Data(1))
    assert calls == [(True, "default")]
    failing[0] = True
    calls.clear()
    sim = LangevinSimulation(device="cpu", compile=True)
    sim.model = Toy()
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        sim.compile_model(Data(3))
    assert any("suppress_errors" in str(x.message) for x in w)
    assert len(calls) == 2 and torch._dynamo.config.suppress_errors
    sim = LangevinSimulation(device="cpu")
    sim.model = Toy()
    d = Data(2)
    d.pos[0, 0] = float("nan")
    with pytest.raises(RuntimeError, match="forces"):
        sim.compile_model(d)
