"""Output network kernels (mlcg_out_forward, mlcg_out_rev2) against float64
torch: values against the module's own arithmetic, the reverse seed adjoint
and the second-order sweep against torch.autograd (jvp for the tangent, then
reverse mode for the force-matching gradients) at ragged row counts.

Every element is held to rtol of the tensor's largest element (check with
atol_frac=1.0): the first layer is a split-operand product on the fp16 MFMA
(about 22 significant bits), whose error scales with the sum of its terms."""

import math

import pytest
import torch

from tests.helpers import check

pytestmark = pytest.mark.gpu


def _act(z, act):
    if act == 0:
        return torch.tanh(z)
    return torch.nn.functional.softplus(z) - math.log(2.0)


def _params(hh, seed, b0=True, b1=False):
    g = torch.Generator(device="cuda").manual_seed(seed)
    W0 = torch.randn(hh, 128, device="cuda", generator=g) / 11
    bb0 = torch.randn(hh, device="cuda", generator=g) if b0 else None
    w1 = torch.randn(1, hh, device="cuda", generator=g) / 8
    bb1 = torch.randn(1, device="cuda", generator=g) if b1 else None
    return W0, bb0, w1, bb1


def _o64(x, W0, b0, w1, b1, act):
    z = x.mm(W0.t())
    if b0 is not None:
        z = z + b0
    o = _act(z, act).mm(w1.t()).view(-1)
    return o + b1 if b1 is not None else o


@pytest.mark.parametrize("rows", [1, 15, 16, 17, 1000, 17920])
@pytest.mark.parametrize("hh,act,b0,b1", [(64, 0, True, False), (64, 1, True, True),
                                          (32, 0, False, True), (128, 1, True, False)])
def test_out_forward(rows, hh, act, b0, b1):
    from mlcg_amd import ops

    print(f"out_forward rows={rows} hh={hh} act={act}", flush=True)
    W0, bb0, w1, bb1 = _params(hh, rows + hh, b0, b1)
    g = torch.Generator(device="cuda").manual_seed(rows)
    x = torch.randn(rows, 128, device="cuda", generator=g)
    seed = torch.randn(rows, device="cuda", generator=g)
    o, oz, os_, xbar = ops.out_forward(x, W0, bb0, w1, bb1, act, seed=seed, reverse=True)
    d = lambda t: None if t is None else t.double()  # noqa: E731
    x64 = x.double().requires_grad_(True)
    o_ref = _o64(x64, d(W0), d(bb0), d(w1), d(bb1), act)
    check(o, o_ref.detach(), 2e-6, 'o', atol_frac=1.0)
    z_ref = x64.detach().mm(d(W0).t()) + (0 if bb0 is None else d(bb0))
    check(os_, _act(z_ref, act), 2e-6, 'os_', atol_frac=1.0)
    if act == 1:
        check(oz, z_ref, 1e-6, 'oz', atol_frac=1.0)
    else:
        assert oz is None
    (xbar_ref,) = torch.autograd.grad((o_ref * seed.double()).sum(), x64, retain_graph=True)
    check(xbar, xbar_ref, 2e-6, 'xbar', atol_frac=1.0)
    # all-ones seed when none is given; no o / no saves on request
    o2, _, _, xbar1 = ops.out_forward(x, W0, bb0, w1, bb1, act, reverse=True, want_o=False,
                                      save=False)
    assert o2 is None
    (xbar1_ref,) = torch.autograd.grad(o_ref.sum(), x64)
    check(xbar1, xbar1_ref, 2e-6, 'xbar1', atol_frac=1.0)


@pytest.mark.parametrize("rows", [1, 17, 1000, 17920])
@pytest.mark.parametrize("hh,act,b0,b1", [(64, 0, True, False), (64, 1, True, True),
                                          (32, 1, False, True), (128, 0, True, True)])
@pytest.mark.parametrize("terms", ["both", "tangent", "primal"])
def test_out_rev2_matches_autograd(rows, hh, act, b0, b1, terms):
    from mlcg_amd import ops

    print(f"out_rev2 rows={rows} hh={hh} act={act} terms={terms}", flush=True)
    W0, bb0, w1, bb1 = _params(hh, 3 * rows + hh, b0, b1)
    g = torch.Generator(device="cuda").manual_seed(rows + 7)
    x = torch.randn(rows, 128, device="cuda", generator=g)
    xdot = torch.randn(rows, 128, device="cuda", generator=g)
    tw = torch.randn(rows, device="cuda", generator=g) if terms != "primal" else None
    pw = torch.randn(rows, device="cuda", generator=g) if terms != "tangent" else None
    _, oz, os_, _ = ops.out_forward(x, W0, bb0, w1, bb1, act)
    use_xdot = terms != "primal"
    odot, xbar2, gW0, gb0, gW1, gb1 = ops.out_rev2(
        x, xdot if use_xdot else None, W0, w1, oz, os_, act, tw, pw, b0, b1,
        want_odot=use_xdot)

    leaves = [t.double().requires_grad_(True) if t is not None else None
              for t in (x, W0, bb0, w1, bb1)]
    x64, W064, b064, w164, b164 = leaves
    f = lambda xx: _o64(xx, W064, b064, w164, b164, act)  # noqa: E731
    o_ref, odot_ref = torch.autograd.functional.jvp(f, (x64,), (xdot.double(),),
                                                    create_graph=True)
    L = 0.0
    if tw is not None:
        L = L + (tw.double() * odot_ref).sum()
    if pw is not None:
        L = L + (pw.double() * o_ref).sum()
    wrt = [t for t in leaves if t is not None]
    grads = torch.autograd.grad(L, wrt, allow_unused=True)
    ref = dict(zip([id(t) for t in wrt], grads))
    z = lambda t: torch.zeros_like(t) if ref[id(t)] is None else ref[id(t)]  # noqa: E731
    if use_xdot:
        check(odot, odot_ref, 2e-6, 'odot', atol_frac=1.0)
    check(xbar2, z(x64), 5e-6, 'xbar2', atol_frac=1.0)
    check(gW0, z(W064), 5e-6, 'gW0', atol_frac=1.0)
    check(gW1, z(w164), 5e-6, 'gW1', atol_frac=1.0)
    if b0:
        check(gb0, z(b064), 5e-6, 'gb0', atol_frac=1.0)
    else:
        assert gb0 is None
    if b1:
        want = z(b164)
        assert float((gb1.double().cpu() - want.cpu()).abs().max()) <= 1e-5 * max(
            1.0, float(want.abs().max()))
    # deterministic: a second call gives identical bits
    again = ops.out_rev2(x, xdot if use_xdot else None, W0, w1, oz, os_, act, tw, pw, b0, b1,
                         want_odot=use_xdot)
    assert torch.equal(again[2], gW0) and torch.equal(again[1], xbar2)


def test_out_kernels_reject_bad_shapes():
    from mlcg_amd import ops

    x = torch.randn(10, 128, device="cuda")
    W0 = torch.randn(48, 128, device="cuda")
    with pytest.raises(RuntimeError):
        ops.out_forward(x, W0, None, torch.randn(1, 48, device="cuda"), None, 0)
