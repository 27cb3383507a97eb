"""The force-matching loss on the HIP kernels (ops.mse_mean and its backward,
used by nn.ForceMSE for the mean of fp32 GPU tensors) against torch's
mse_loss: the loss to rounding (the summation orders differ), the gradient
bit for bit (the same expression), one and several 64 Ki-element chunks."""

import pytest
import torch
from torch.nn import functional as F

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 7, 53760, 65536, 65537, 3_000_001])
def test_mse_mean_matches_torch(n):
    from mlcg_amd import ops
    from mlcg_amd.nn.losses import _mse

    print(f"mse_mean n={n}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(n)
    x = torch.randn(n, device="cuda", generator=g)
    y = torch.randn(n, device="cuda", generator=g)
    ref64 = ((x.double() - y.double()) ** 2).mean()
    loss = ops.mse_mean(x, y)
    assert loss.shape == () and loss.dtype == torch.float32
    assert abs(float(loss) - float(ref64)) <= 2e-6 * abs(float(ref64))
    assert float(loss) == float(ops.mse_mean(x, y))  # fixed order: run-to-run identical
    xa = x.clone().requires_grad_(True)
    xb = x.clone().requires_grad_(True)
    seed = torch.tensor(0.37, device="cuda")
    _mse(xa, y, "mean").backward(seed)
    F.mse_loss(xb, y).backward(seed)
    assert torch.equal(xa.grad, xb.grad)


def test_force_mse_module_paths():
    """nn.ForceMSE takes the kernels for its mean and falls back to torch for
    the other reductions, for fp64 data and for targets that need gradients."""
    from mlcg_amd import nn
    from mlcg_amd.nn.losses import _MSEMean, _mse

    g = torch.Generator(device="cuda").manual_seed(3)
    f = torch.randn(100, 3, device="cuda", generator=g, requires_grad=True)
    r = torch.randn(100, 3, device="cuda", generator=g)
    out = _mse(f, r, "mean")
    assert out.grad_fn is not None and isinstance(out.grad_fn, _MSEMean._backward_cls)
    for red in ("sum", "none"):
        assert torch.equal(_mse(f, r, red), F.mse_loss(f, r, reduction=red))
    f64, r64 = f.detach().double().requires_grad_(True), r.double()
    assert torch.equal(_mse(f64, r64, "mean"), F.mse_loss(f64, r64))
    rg = r.clone().requires_grad_(True)
    assert torch.equal(_mse(f, rg, "mean"), F.mse_loss(f, rg))
    assert isinstance(nn.ForceMSE(), torch.nn.Module)
