"""Training-step integration (mlcg/pl/model.py:19-131): the Lightning-free
PLModel on a toy model whose forces are known in closed form (CPU), and on
the fused SchNet against the plain model -> loss -> backward -> AdamW path
(GPU)."""

import pytest
import torch
import torch.nn.functional as Fn

from mlcg_amd.data import AtomicData
from mlcg_amd.data.atomic_data import collate
from mlcg_amd.nn import ForceMSE, GradientsOut, Loss
from mlcg_amd.pl import PLModel, detect_nan_parameters, train_epoch


class HarmonicToy(torch.nn.Module):
    """E_b = k/2 sum_{n in b} |x_n|^2, so F = -k x."""

    name = "Toy"

    def __init__(self, k=1.0):
        super().__init__()
        self.k = torch.nn.Parameter(torch.tensor(float(k)))

    def forward(self, data):
        e = 0.5 * self.k * (data.pos * data.pos).sum(1)
        E = torch.zeros(int(data.n_atoms.shape[0]), dtype=e.dtype).index_add(0, data.batch, e)
        data.out[self.name] = {"energy": E}
        return data


def _batch(sizes, k_true=2.5, seed=0):
    g = torch.Generator().manual_seed(seed)
    frames = []
    for n in sizes:
        x = torch.randn(n, 3, generator=g)
        frames.append(AtomicData.from_points(x, torch.arange(n), forces=-k_true * x))
    return collate(frames)


def test_step_loss_batch_size_and_log():
    pl = PLModel(GradientsOut(HarmonicToy(1.0)), Loss([ForceMSE()]))
    assert pl.derivative
    data = _batch([3, 5, 4])
    ref_pos = data.pos.clone()
    loss, bs = pl.step(data, "train")
    assert bs == 3
    assert torch.allclose(loss, Fn.mse_loss(-1.0 * ref_pos, -2.5 * ref_pos))
    assert torch.equal(pl.logged["train_loss"], loss.detach())
    assert loss.requires_grad
    # outputs of the wrapped model are merged into data.out (model.py:116)
    assert "forces" in data.out and "energy" in data.out


def test_validation_epoch_end_is_the_reference_weighted_mean():
    pl = PLModel(GradientsOut(HarmonicToy(1.0)), Loss([ForceMSE()]))
    losses = []
    for i, sizes in enumerate(([3, 4], [5], [2, 2, 2])):
        loss, bs = pl.validation_step(_batch(sizes, seed=i), i)
        losses.append((loss.item(), bs))
    out = pl.on_validation_epoch_end()
    # one metaset: weights b / sum_metasets(b) = 1, then the mean over batches
    assert out.item() == pytest.approx(sum(l for l, _ in losses) / 3, rel=1e-12)
    assert pl.validation_step_outputs == []
    assert pl.logged["validation_loss"].item() == pytest.approx(out.item())


def test_train_epoch_fits_the_spring_constant():
    pl = PLModel(GradientsOut(HarmonicToy(0.5)), Loss([ForceMSE()]))
    opt = pl.configure_optimizers(lr=0.05)
    assert isinstance(opt, torch.optim.AdamW)
    batches = [_batch([4, 6], seed=s) for s in range(4)]
    first = train_epoch(pl, batches, opt)
    for _ in range(40):
        last = train_epoch(pl, batches, opt)
    assert last < 1e-3 * first
    assert pl.model.model.k.item() == pytest.approx(2.5, rel=1e-2)


def test_detect_nan_parameters_and_get_model():
    toy = HarmonicToy(1.0)
    pl = PLModel(GradientsOut(toy), Loss([ForceMSE()]))
    copy = pl.get_model()
    assert copy is not pl.model and copy.model.k.item() == 1.0
    detect_nan_parameters(toy)
    with torch.no_grad():
        toy.k.fill_(float("nan"))
    with pytest.raises(ValueError, match="k"):
        pl.on_train_epoch_end()


@pytest.mark.gpu
def test_plmodel_step_matches_the_plain_training_step():
    """PLModel.training_step + AdamW on the fused SchNet gives the same loss,
    gradients and updated parameters as model -> ForceMSE -> backward ->
    AdamW written out by hand (the path bench.py times)."""
    from mlcg_amd import synthetic
    from oracle import schnet_ref as R
    from tests.helpers import make_cfg, make_model

    cfg = make_cfg(num_blocks=2, rc=20.0)
    sd = R.random_state_dict(cfg, seed=21)
    b = synthetic.config2(n_frames=8)
    b.forces = (0.1 * torch.randn(b.pos.shape, generator=torch.Generator().manual_seed(2))
                ).numpy()
    models = [make_model(cfg, sd) for _ in range(2)]
    for m in models:
        m.train()
    pl = PLModel(GradientsOut(models[0]), Loss([ForceMSE()])).to("cuda")  # as Lightning does
    opt_pl = pl.configure_optimizers(lr=1e-3)
    plain = GradientsOut(models[1])
    opt = torch.optim.AdamW(models[1].parameters(), lr=1e-3, weight_decay=0.0, fused=True)
    for it in range(2):
        train_epoch(pl, [b.to_torch("cuda")], opt_pl)
        opt.zero_grad(set_to_none=True)
        data = plain(b.to_torch("cuda"))
        data.out.update(**data.out[plain.name])
        loss = ForceMSE()(data)
        loss.backward()
        opt.step()
        assert torch.equal(pl.logged["train_loss"], loss.detach())
        for (n0, p0), (n1, p1) in zip(models[0].named_parameters(),
                                      models[1].named_parameters()):
            assert n0 == n1
            assert torch.equal(p0, p1), (it, n0)  # every reduction has a fixed order


@pytest.mark.gpu
def test_plmodel_step_against_oracle_gradients_and_cpu_adamw():
    """Two PLModel training steps (pl/model.py:113-131 + AdamW) on the fused
    SchNet: at each step the loss and every parameter gradient match the fp64
    oracle's force_matching_grads evaluated at the step's parameters (rtol
    1e-4 per element), and the AdamW update equals torch's CPU AdamW in fp64
    applied to the same gradients (rtol 1e-6)."""
    from mlcg_amd import synthetic
    from oracle import radius as oracle_radius
    from oracle import schnet_ref as R
    from tests.helpers import check, make_cfg, make_model

    cfg = make_cfg(num_blocks=2, rc=20.0)
    sd = R.random_state_dict(cfg, seed=22)
    b = synthetic.config2(n_frames=8)
    model = make_model(cfg, sd).train()
    pl = PLModel(GradientsOut(model), Loss([ForceMSE()])).to("cuda")
    opt = pl.configure_optimizers(lr=1e-3, weight_decay=0.01)
    group = opt.param_groups[0]
    names = [n for n, _ in model.named_parameters()]
    cpu_params = [p.detach().double().cpu().clone().requires_grad_(False)
                  for p in model.parameters()]
    cpu_opt = torch.optim.AdamW(cpu_params, lr=group["lr"], betas=group["betas"],
                                eps=group["eps"], weight_decay=group["weight_decay"])
    ei, _ = oracle_radius.radius_graph(b.pos, 20.0, b.batch, False, 1000)
    args = (torch.from_numpy(b.pos).double(), torch.from_numpy(b.atom_types),
            torch.from_numpy(b.batch), torch.from_numpy(ei), b.n_frames,
            torch.from_numpy(b.forces).double())
    for step in range(2):
        # the oracle at the parameters this step starts from
        sd_now = {k: v.detach().double().cpu() for k, v in model.state_dict().items()}
        loss_ref, _, _, g_ref = R.force_matching_grads(sd_now, cfg, *args)
        train_epoch(pl, [b.to_torch("cuda")], opt)
        got_loss = float(pl.logged["train_loss"])
        assert abs(got_loss - float(loss_ref)) <= 1e-5 * abs(float(loss_ref)), step
        grads = {n: p.grad.detach().double().cpu() for n, p in model.named_parameters()}
        for n in names:
            check(grads[n], g_ref[n], 1e-4, f"step {step} grad {n}")
        # CPU AdamW (fp64) fed the same gradients the GPU step used
        for n, p in zip(names, cpu_params):
            p.grad = grads[n].clone()
        cpu_opt.step()
        for n, p_gpu, p_cpu in zip(names, model.parameters(), cpu_params):
            check(p_gpu.detach(), p_cpu, 1e-6, f"step {step} AdamW update {n}")
            p_cpu.copy_(p_gpu.detach().double().cpu())  # continue from the GPU state
