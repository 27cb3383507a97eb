"""Node-level weight-gradient reduction (mlcg_node_tmm) against fp64 torch
products at ragged row counts, and the node_linear helper's epilogues."""

import pytest
import torch

from tests.helpers import rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("transpose", [False, True])
def test_node_linear_helper(transpose):
    from mlcg_amd import ops

    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(1000, 128, device="cuda", generator=g)
    W = torch.randn(128, 128, device="cuda", generator=g) / 11
    b = torch.randn(128, device="cuda", generator=g)
    r = torch.randn(1000, 128, device="cuda", generator=g)
    Wd = W.double()
    ref = x.double().mm(Wd if transpose else Wd.t())
    assert rel_err(ops.node_linear(x, W, transpose=transpose), ref) < 1e-6
    out = ops.node_linear(x, W, bias=b, residual=r, transpose=transpose)
    assert rel_err(out, ref + b.double() + r.double()) < 1e-6


@pytest.mark.parametrize("rows", [0, 1, 127, 128, 129, 5000, 17920])
def test_node_tmm(rows):
    from mlcg_amd import ops

    g = torch.Generator(device="cuda").manual_seed(rows + 1)
    a1, b1, a2, b2 = (torch.randn(rows, 128, device="cuda", generator=g) for _ in range(4))
    ref = a1.double().t().mm(b1.double())
    got = ops.node_tmm(a1, b1)
    if rows == 0:
        assert float(got.abs().max()) == 0.0
        return
    assert rel_err(got, ref) < 1e-6
    ref2 = ref + a2.double().t().mm(b2.double())
    assert rel_err(ops.node_tmm(a1, b1, a2, b2), ref2) < 1e-6
    # deterministic: bitwise identical on a second call
    assert torch.equal(ops.node_tmm(a1, b1, a2, b2), ops.node_tmm(a1, b1, a2, b2))
