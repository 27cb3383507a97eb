"""The force-matching training step captured as one HIP graph (bench.py's
captured_step) against the same step run eagerly: every replay, with eager
work and synchronisations between the replays, gives the eager loss and
parameters bit for bit.  The capture follows torch's rules: a capturable
optimizer (a non-capturable one raises inside the capture region), warm-up
and capture on one side stream, no timing events inside the capture."""

import pytest
import torch

from oracle import schnet_ref as R
from tests.helpers import make_cfg, make_model

pytestmark = pytest.mark.gpu


def test_captured_training_step_matches_eager():
    from mlcg_amd import nn, synthetic

    print("captured training step, 2 blocks, 16 frames", flush=True)
    cfg = make_cfg(num_blocks=2, rc=20.0)
    sd = R.random_state_dict(cfg, seed=31)
    b = synthetic.config2(n_frames=16)
    b.forces = (0.1 * torch.randn(b.pos.shape, generator=torch.Generator().manual_seed(4))
                ).numpy()
    runs = []
    for capture in (False, True):
        model = make_model(cfg, sd).train()
        data = b.to_torch("cuda")
        g0 = model.build_graph(data)
        model.graph_capacity = int(g0.num_edges * 1.05) + 64 + (int(g0.num_edges * 1.05) % 2)
        gm = nn.GradientsOut(model)
        opt = torch.optim.AdamW(model.parameters(), lr=1e-3, fused=True, capturable=True)

        def step():
            opt.zero_grad(set_to_none=True)
            out = gm(data)
            out.out.update(**out.out[model.name])
            loss = nn.ForceMSE()(out)
            loss.backward()
            opt.step()
            return loss

        losses, params = [], []
        if capture:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                losses.append(step().detach().clone())  # eager steps 1, 2
                params.append([p.detach().clone() for p in model.parameters()])
                losses.append(step().detach().clone())
                params.append([p.detach().clone() for p in model.parameters()])
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                static_loss = step()
            for _ in range(4):  # steps 3..6 by replay, eager work in between
                graph.replay()
                junk = torch.randn(1000, 128, device="cuda").sum()
                torch.cuda.synchronize()
                losses.append(static_loss.detach().clone())
                params.append([p.detach().clone() for p in model.parameters()])
                del junk
        else:
            for _ in range(6):
                losses.append(step().detach().clone())
                params.append([p.detach().clone() for p in model.parameters()])
        runs.append((losses, params))
    (le, pe), (lg, pg) = runs
    for k in range(6):
        assert torch.equal(le[k], lg[k]), k
        for a, c in zip(pe[k], pg[k]):
            assert torch.equal(a, c), k


def _step_run(cfg, sd, b, ahead, tmm_side, n_steps=3, captured=False, capturable=False):
    """Losses, forces and parameters after each of n_steps training steps
    with the given stream arrangement (eager), or through CapturedTrainStep
    (which needs the capturable AdamW)."""
    from mlcg_amd import nn
    from mlcg_amd.nn import _fused
    from mlcg_amd.pl import CapturedTrainStep

    saved = _fused._FILTER_AHEAD, _fused._TMM_SIDE
    _fused._FILTER_AHEAD, _fused._TMM_SIDE = ahead, tmm_side
    try:
        model = make_model(cfg, sd).train()
        data = b.to_torch("cuda")
        g0 = model.build_graph(data)
        cap = int(g0.num_edges * 1.05) + 64
        model.graph_capacity = cap + (cap % 2)
        gm = nn.GradientsOut(model)
        opt = torch.optim.AdamW(model.parameters(), lr=1e-3, fused=True,
                                capturable=captured or capturable)
        forces = []

        def step(d):
            opt.zero_grad(set_to_none=True)
            out = gm(d)
            out.out.update(**out.out[model.name])
            forces.append(out.out["forces"].detach().clone())
            loss = nn.ForceMSE()(out)
            loss.backward()
            opt.step()
            return loss

        losses, params = [], []
        if captured:
            cs = CapturedTrainStep(step, data, model, opt, warmup=1)  # eager step 1
            losses.append(None)
            params.append(None)
            batch = b.to_torch("cuda")  # a second resident copy, loaded each step
            for _ in range(n_steps - 1):
                loss = cs.step(batch)
                torch.cuda.synchronize()
                losses.append(loss.detach().clone())
                params.append([p.detach().clone() for p in model.parameters()])
            cs.check()
        else:
            for _ in range(n_steps):
                losses.append(step(data).detach().clone())
                params.append([p.detach().clone() for p in model.parameters()])
        return losses, forces, params
    finally:
        _fused._FILTER_AHEAD, _fused._TMM_SIDE = saved


def test_stream_arrangements_bit_identical():
    """The filter forwards issued ahead on the side stream, and the
    weight-gradient reductions on the side stream, change only where kernels
    run, never what they compute: every arrangement gives the in-order
    single-stream step's losses, forces and parameters bit for bit."""
    from mlcg_amd import synthetic

    print("stream arrangements, 3 blocks, 16 frames", flush=True)
    cfg = make_cfg(num_blocks=3, rc=20.0)
    sd = R.random_state_dict(cfg, seed=32)
    b = synthetic.config2(n_frames=16)
    ref = _step_run(cfg, sd, b, ahead=False, tmm_side=False)
    for ahead, side in ((True, False), (False, True), (True, True)):
        got = _step_run(cfg, sd, b, ahead=ahead, tmm_side=side)
        for k in range(3):
            assert torch.equal(got[0][k], ref[0][k]), (ahead, side, k)
            assert torch.equal(got[1][k], ref[1][k]), (ahead, side, k)
            for a, c in zip(got[2][k], ref[2][k]):
                assert torch.equal(a, c), (ahead, side, k)


def test_node_weight_images_step_bit_identical():
    """Training steps whose node products read the per-forward split weight
    images give the losses, forces and parameters of steps whose products
    split the weights in every launch, bit for bit."""
    from mlcg_amd import synthetic
    from mlcg_amd.nn import _fused

    print("weight images vs in-kernel splits, 3 blocks, 16 frames", flush=True)
    cfg = make_cfg(num_blocks=3, rc=20.0)
    sd = R.random_state_dict(cfg, seed=35)
    b = synthetic.config2(n_frames=16)
    saved = _fused._NODE_IMAGES
    try:
        _fused._NODE_IMAGES = False
        ref = _step_run(cfg, sd, b, ahead=True, tmm_side=False)
        _fused._NODE_IMAGES = True
        got = _step_run(cfg, sd, b, ahead=True, tmm_side=False)
    finally:
        _fused._NODE_IMAGES = saved
    for k in range(3):
        assert torch.equal(got[0][k], ref[0][k]), k
        assert torch.equal(got[1][k], ref[1][k]), k
        for a, c in zip(got[2][k], ref[2][k]):
            assert torch.equal(a, c), k


def test_captured_train_step_api_matches_eager():
    """mlcg_amd.pl.CapturedTrainStep (one warm-up step, then replays that
    each load a second resident copy of the batch) gives the eager steps'
    losses and parameters bit for bit, with the filter forwards ahead on the
    side stream inside the graph."""
    from mlcg_amd import synthetic

    print("CapturedTrainStep, 3 blocks, 16 frames", flush=True)
    cfg = make_cfg(num_blocks=3, rc=20.0)
    sd = R.random_state_dict(cfg, seed=33)
    b = synthetic.config2(n_frames=16)
    ref = _step_run(cfg, sd, b, ahead=True, tmm_side=True, n_steps=4, capturable=True)
    got = _step_run(cfg, sd, b, ahead=True, tmm_side=True, n_steps=4, captured=True)
    for k in range(1, 4):
        assert torch.equal(got[0][k], ref[0][k]), k
        for a, c in zip(got[2][k], ref[2][k]):
            assert torch.equal(a, c), k


def test_captured_train_step_overflow_raises_at_check():
    """A batch with more edges than the captured step's edge capacity does not
    grow the graph: the replays run on the truncated graph (every kernel
    stays inside its buffers) and check() raises naming the capacity; the
    flags are cleared by the raising check."""
    from mlcg_amd import nn, synthetic
    from mlcg_amd.pl import CapturedTrainStep

    print("CapturedTrainStep with half the needed edge capacity", flush=True)
    cfg = make_cfg(num_blocks=2, rc=20.0)
    sd = R.random_state_dict(cfg, seed=36)
    model = make_model(cfg, sd).train()
    data = synthetic.config2(n_frames=4).to_torch("cuda")
    gm = nn.GradientsOut(model)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3, fused=True, capturable=True)

    def step(d):
        opt.zero_grad(set_to_none=True)
        out = gm(d)
        out.out.update(**out.out[model.name])
        loss = nn.ForceMSE()(out)
        loss.backward()
        opt.step()
        return loss

    e_full = model.build_graph(data).num_edges
    cs = CapturedTrainStep(step, data, model, opt, warmup=1, capacity_factor=0.5)
    assert 0 < model.graph_capacity < e_full
    cs.step(data)
    cs.step(data)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="more edges than the capacity"):
        cs.check()
    cs.check()  # cleared by the raising check


def test_captured_train_step_requires_capturable_optimizer():
    from mlcg_amd import nn, synthetic
    from mlcg_amd.pl import CapturedTrainStep

    cfg = make_cfg(num_blocks=1, rc=20.0)
    sd = R.random_state_dict(cfg, seed=34)
    model = make_model(cfg, sd).train()
    data = synthetic.config2(n_frames=2).to_torch("cuda")
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
    with pytest.raises(RuntimeError, match="capturable"):
        CapturedTrainStep(lambda d: nn.GradientsOut(model)(d), data, model, opt)
