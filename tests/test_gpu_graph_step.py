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
