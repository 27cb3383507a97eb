"""Range guards of the split-fp16 products (filter.hip).

The split filter forward carries per-pair activations h = act(a) and their
distance derivatives h' as fp16 hi/lo pairs, which hold |h| < 2^15; a tile
whose values pass that bound is recomputed with a power-of-two scale, so the
result stays exact.  The split filter backward holds |h| < 2^19 and sets bit 0
of mlcg_numerics_flags beyond it; ops.check_numerics raises, and the strict
fp32 filters (forward and backward on the fp32 MFMA) handle such models.

The models are shifted-softplus SchNets whose first filter layer is scaled up
(pre-activations of order 10^5 and 10^6, so h = softplus(a) - ln 2 ~ a) and
whose second layer is scaled down by the same factor, so the filters and
everything downstream stay of order one.  Energies, forces and parameter
gradients are compared with the fp64 oracle (oracle/schnet_ref.py), the bound
widened where the reference's own fp32 arithmetic needs it (check_calibrated).
"""

import pytest
import torch

from oracle import schnet_ref as R
from tests.helpers import check_calibrated, make_cfg, make_model
from tests.test_gpu_schnet import _oracle_inputs, _small_batch

pytestmark = pytest.mark.gpu

RC = 12.0


def _scaled_sd(scale, seed, bias_shift=0.0):
    """First filter layer times `scale` (plus `bias_shift` on its bias),
    second layer divided by scale (by bias_shift when that is larger)."""
    cfg = make_cfg(num_blocks=2, rc=RC, act="ssp")
    sd = R.random_state_dict(cfg, seed=seed)
    for k in range(cfg.num_blocks):
        pre = f"interaction_blocks.{k}.conv.filter_network.layers"
        sd[f"{pre}.0.weight"] = sd[f"{pre}.0.weight"] * scale
        sd[f"{pre}.0.bias"] = sd[f"{pre}.0.bias"] * scale + bias_shift
        sd[f"{pre}.2.weight"] = sd[f"{pre}.2.weight"] / max(scale, bias_shift)
    return cfg, sd


def _max_preactivation(cfg, sd, pos64, ei):
    """Largest a = W1 g(d) + b1 over the graph's pairs and the blocks (fp64);
    shifted softplus makes h = a - ln 2 + O(e^-a) of the positive ones."""
    sd64 = R.to_dtype(sd, torch.float64)
    d = (pos64[ei[1]] - pos64[ei[0]]).norm(dim=1)
    g = R.gaussian_rbf(d, sd64["rbf_layer.offset"], sd64["rbf_layer.coeff"],
                       R.Cutoff("cosine", 0.0, RC))
    m = 0.0
    for k in range(cfg.num_blocks):
        pre = f"interaction_blocks.{k}.conv.filter_network.layers.0"
        a = g @ sd64[f"{pre}.weight"].t() + sd64[f"{pre}.bias"]
        m = max(m, float(a.max()))
    return m


def test_split_forward_large_activations_exact():
    """Activations of ~10^5 (past the split forward's 2^15): energies and
    forces still match the fp64 oracle, finite, with no flag raised."""
    from mlcg_amd import nn, ops

    print("split forward, activations past 2^15", flush=True)
    cfg, sd = _scaled_sd(2.0e5, seed=21)
    b = _small_batch()
    pos64, types, batch, ei = _oracle_inputs(b, RC)
    amax = _max_preactivation(cfg, sd, pos64, ei)
    print(f"largest pre-activation {amax:.3e}")
    assert amax > 2.0 ** 16
    E_ref, F_ref = R.schnet_energy_forces(R.to_dtype(sd, torch.float64), cfg, pos64, types,
                                          batch, ei, b.n_frames)
    E32, F32 = R.schnet_energy_forces(sd, cfg, pos64.float(), types, batch, ei, b.n_frames)
    model = make_model(cfg, sd)
    ops.numerics_flags(clear=True)
    data = nn.GradientsOut(model).eval()(b.to_torch("cuda"))
    E, F = data.out["SchNet"]["energy"], data.out["SchNet"]["forces"]
    assert bool(torch.isfinite(E).all()) and bool(torch.isfinite(F).all())
    check_calibrated(E, E_ref, E32, 1e-5, "E")
    check_calibrated(F, F_ref, F32, 1e-5, "F")
    ops.check_numerics()


def _train_grads(cfg, sd, b, strict):
    from mlcg_amd import nn

    model = make_model(cfg, sd)
    model.strict_fp32_filters = strict
    data = nn.GradientsOut(model).train()(b.to_torch("cuda"))
    loss = torch.nn.functional.mse_loss(data.out["SchNet"]["forces"], data.forces)
    loss.backward()
    torch.cuda.synchronize()
    return loss, {k: p.grad for k, p in model.named_parameters()}


def test_split_backward_range_flag_and_strict_path():
    """Activations of ~10^6 (past the split backward's 2^19; from the first
    layer's bias, the weights stay of order one): the training step raises
    through ops.check_numerics instead of handing back unreported non-finite
    gradients; with strict fp32 filters (forward and backward on the fp32
    MFMA) no flag is raised and every parameter gradient matches the fp64
    oracle."""
    from mlcg_amd import ops

    print("split backward, activations past 2^19", flush=True)
    cfg, sd = _scaled_sd(1.0, seed=22, bias_shift=2.0e6)
    b = _small_batch()
    pos64, types, batch, ei = _oracle_inputs(b, RC)
    amax = _max_preactivation(cfg, sd, pos64, ei)
    print(f"largest pre-activation {amax:.3e}")
    assert amax > 2.0 ** 20
    ops.numerics_flags(clear=True)
    _train_grads(cfg, sd, b, strict=False)
    with pytest.raises(RuntimeError, match="2\\^19"):
        ops.check_numerics()
    ops.check_numerics()  # cleared by the raising check
    loss, grads = _train_grads(cfg, sd, b, strict=True)
    ops.check_numerics()
    fref64 = torch.from_numpy(b.forces).double()
    loss_ref, _, _, g_ref = R.force_matching_grads(R.to_dtype(sd, torch.float64), cfg, pos64,
                                                   types, batch, ei, b.n_frames, fref64)
    _, _, _, g32 = R.force_matching_grads(sd, cfg, pos64.float(), types, batch, ei, b.n_frames,
                                          fref64.float())
    assert abs(float(loss) - float(loss_ref)) <= 1e-5 * abs(float(loss_ref))
    for k, gr in g_ref.items():
        got = grads[k]
        assert got is not None and bool(torch.isfinite(got).all()), k
        check_calibrated(got, gr, g32[k], 1e-4, k)


def test_split_weight_range_flag():
    """A first-layer weight past 65504 (the fp16 maximum): the split kernels
    flag it (forward and backward) and ops.check_numerics raises; strict fp32
    filters raise no flag."""
    from mlcg_amd import ops

    print("split kernels, weights past the fp16 maximum", flush=True)
    cfg, sd = _scaled_sd(1.0e6, seed=23)
    b = _small_batch()
    ops.numerics_flags(clear=True)
    _train_grads(cfg, sd, b, strict=False)
    with pytest.raises(RuntimeError, match="fp16 maximum"):
        ops.check_numerics()
    _train_grads(cfg, sd, b, strict=True)
    ops.check_numerics()


def test_numerics_flags_capturable_read():
    """The flag reader only enqueues a kernel (no host synchronisation), so
    it can sit inside a captured training step."""
    from mlcg_amd import ops

    ops.numerics_flags(clear=True)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = ops.numerics_flags(clear=False)
        with torch.cuda.graph(g, stream=s):
            out = ops.numerics_flags(clear=False)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert int(out.item()) == 0
