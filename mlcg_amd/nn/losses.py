"""Losses (mlcg/nn/losses.py:11-181)."""

from __future__ import annotations

from typing import List, Optional

import torch
from torch.nn import functional as F
from torch.nn.modules.loss import _Loss

from .. import ops
from ..data._keys import ENERGY_KEY, FORCE_KEY


class Loss(torch.nn.Module):
    def __init__(self, losses: List[_Loss], weights: Optional[List[float]] = None) -> None:
        super().__init__()
        weights = torch.ones(len(losses)) if weights is None else torch.tensor(weights)
        assert len(weights) == len(losses)
        self.register_buffer("weights", weights)
        self.losses = losses

    def forward(self, data) -> torch.Tensor:
        loss = torch.zeros((len(self.losses)), device=self.weights.device)
        for ii, loss_fn in enumerate(self.losses):
            loss[ii] = loss_fn(data) * self.weights[ii]
        return loss.sum()


def _check(data, kwd):
    if kwd not in data.out:
        raise RuntimeError(
            f"target property {kwd} has not been computed in data.out {list(data.out.keys())}")
    if kwd not in data:
        raise RuntimeError(f"target property {kwd} has no reference in data {data.keys()}")


class ForceRMSE(_Loss):
    def __init__(self, force_kwd: str = FORCE_KEY, size_average=None, reduce=None,
                 reduction: str = "mean") -> None:
        super().__init__(size_average=size_average, reduce=reduce, reduction=reduction)
        self.force_kwd = force_kwd

    def forward(self, data) -> torch.Tensor:
        _check(data, self.force_kwd)
        return torch.sqrt(F.mse_loss(data.out[self.force_kwd], data[self.force_kwd],
                                     reduction=self.reduction))


class _MSEMean(torch.autograd.Function):
    """mean((pred - ref)^2) on the HIP kernels (two launches per training step
    instead of torch's five: square, mean, and the backward's zero fill,
    product and seed); the gradient equals torch's mse_loss gradient bit for
    bit, the loss agrees with it to rounding (fixed summation order)."""

    @staticmethod
    def forward(ctx, pred, ref):
        ctx.save_for_backward(pred, ref)
        return ops.mse_mean(pred, ref)

    @staticmethod
    def backward(ctx, grad):
        pred, ref = ctx.saved_tensors
        return ops.mse_mean_backward(pred, ref, grad), None


def _mse(pred: torch.Tensor, ref: torch.Tensor, reduction: str) -> torch.Tensor:
    """F.mse_loss, on the HIP kernels for the training step's case (mean of
    contiguous fp32 GPU tensors, reference without gradient)."""
    if reduction == "mean" and not ref.requires_grad and ops._mse_ok(pred, ref):
        return _MSEMean.apply(pred, ref)
    return F.mse_loss(pred, ref, reduction=reduction)


class ForceMSE(_Loss):
    def __init__(self, force_kwd: str = FORCE_KEY, size_average=None, reduce=None,
                 reduction: str = "mean") -> None:
        super().__init__(size_average=size_average, reduce=reduce, reduction=reduction)
        self.force_kwd = force_kwd

    def forward(self, data) -> torch.Tensor:
        _check(data, self.force_kwd)
        return _mse(data.out[self.force_kwd], data[self.force_kwd], self.reduction)


class EnergyMSE(_Loss):
    def __init__(self, energy_kwd: str = ENERGY_KEY, size_average=None, reduce=None,
                 reduction: str = "mean") -> None:
        super().__init__(size_average=size_average, reduce=reduce, reduction=reduction)
        self.energy_kwd = energy_kwd

    def forward(self, data) -> torch.Tensor:
        _check(data, self.energy_kwd)
        return F.mse_loss(data.out[self.energy_kwd], data[self.energy_kwd],
                          reduction=self.reduction)
