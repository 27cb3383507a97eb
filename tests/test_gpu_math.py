"""The library's own fp32 elementary functions (common.h: tanh, sigmoid,
softplus, sin(pi u), cos(pi u) on the hardware exp2 / log2 / reciprocal with
fitted polynomial parts), evaluated through mlcg_math_eval on dense fp32
grids and compared with fp64 of the same fp32 inputs.  They run inline in the
filter, node and output-network kernels (tanh is the reference's default
activation, schnet.py:419; sigmoid and softplus make the shifted softplus;
sin/cos(pi u) the cosine cutoff, cutoff.py:145-153).

Bounds (measured on MI355X, with some margin):
  tanh     relative <= 2e-7 over [-12, 12] and |x| in [1e-10, 10]
  sigmoid  absolute <= 1.5e-7 (an ulp of 1) over [-90, 90]; relative <= 5e-6
           (the exp2 argument's rounding, |x| 2^-24 log2 e, dominates for
           large |x|, where the value itself is below 1e-6)
  softplus absolute <= 6e-7 (a quarter ulp at 20) over [-90, 30]; relative
           <= 5e-6 (as the sigmoid)
  sin(pi u), cos(pi u)  absolute <= 2e-7 over [-8, 8]; sin(pi k) = 0 and
           |cos(pi k)| = 1 exactly at the integers
torch's own fp32 functions on the same grids are printed for comparison.
"""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu

TANH, SIGMOID, SOFTPLUS, SINPI, COSPI = range(5)


def _eval(fn, x):
    from mlcg_amd import _lib

    y = torch.empty_like(x)
    st = _lib.load().mlcg_math_eval(fn, _lib.ptr(x), x.numel(), _lib.ptr(y),
                                    _lib.stream_handle())
    assert st == 0
    torch.cuda.synchronize()
    return y


def _errors(fn, x32, ref64, torch32):
    y = _eval(fn, x32).double().cpu()
    t = ref64(x32.double().cpu())
    yt = torch32(x32).double().cpu()
    ae, aet = (y - t).abs(), (yt - t).abs()
    nz = t.abs() >= 2.0 ** -126  # relative errors where fp32 is normal
    re = ae[nz] / t.abs()[nz]
    ret = aet[nz] / t.abs()[nz]
    print(f"fn {fn}: abs {float(ae.max()):.3e} rel {float(re.max()):.3e} | torch fp32 abs "
          f"{float(aet.max()):.3e} rel {float(ret.max()):.3e}")
    return float(ae.max()), float(re.max()), y


def test_tanh_accuracy():
    x = torch.cat([torch.linspace(-12, 12, 4_000_001), torch.logspace(-10, 1, 200_001),
                   -torch.logspace(-10, 1, 200_001)]).float().cuda()
    ae, re, y = _errors(TANH, x, torch.tanh, torch.tanh)
    assert re <= 2e-7
    # odd, and saturated to exactly +-1
    xs = torch.linspace(0, 12, 10001).float().cuda()
    assert torch.equal(_eval(TANH, -xs), -_eval(TANH, xs))
    assert float(_eval(TANH, torch.tensor([20.0, -20.0, 88.0], device="cuda")).abs().min()) == 1.0


def test_sigmoid_accuracy():
    x = torch.linspace(-90, 90, 4_000_001).float().cuda()
    ae, re, _ = _errors(SIGMOID, x, torch.sigmoid, torch.sigmoid)
    assert ae <= 1.5e-7 and re <= 5e-6
    assert float(_eval(SIGMOID, torch.zeros(1, device="cuda"))) == 0.5


def test_softplus_accuracy():
    x = torch.cat([torch.linspace(-90, 30, 4_000_001),
                   torch.linspace(-1, 1, 1_000_001)]).float().cuda()
    sp = torch.nn.functional.softplus
    ae, re, _ = _errors(SOFTPLUS, x, sp, sp)
    assert ae <= 6e-7 and re <= 5e-6
    assert abs(float(_eval(SOFTPLUS, torch.zeros(1, device="cuda"))) - math.log(2.0)) <= 6e-8


@pytest.mark.parametrize("fn", [SINPI, COSPI], ids=["sinpi", "cospi"])
def test_sincospi_accuracy(fn):
    x = torch.linspace(-8, 8, 4_000_001).float().cuda()
    ref = (lambda u: torch.sin(math.pi * u)) if fn == SINPI else (lambda u: torch.cos(math.pi * u))
    ae, _, _ = _errors(fn, x, ref, ref)
    assert ae <= 2e-7
    k = torch.arange(-8, 9, dtype=torch.float32, device="cuda")
    if fn == SINPI:
        assert bool((_eval(SINPI, k) == 0).all())
    else:
        assert torch.equal(_eval(COSPI, k).abs(), torch.ones_like(k))
