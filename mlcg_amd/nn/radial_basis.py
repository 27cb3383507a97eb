"""Radial bases: Gaussian (mlcg/nn/radial_basis/gaussian.py:9-102) and
exponential-normal (exp_normal.py:9-178), with the base class of base.py:4-41.
Same constructors, parameter/buffer names and state_dict keys as the
reference; the fused SchNet path evaluates both inside the filter kernel."""

from typing import Union

import torch
from torch import nn

from .cutoff import CosineCutoff, IdentityCutoff, _Cutoff


class _RadialBasis(nn.Module):
    def __init__(self):
        super().__init__()
        self.cutoff = None

    def check_cutoff(self):
        if self.cutoff.cutoff_upper < self.cutoff.cutoff_lower:
            raise ValueError("Upper cutoff {} is less than lower cutoff {}".format(
                self.cutoff.cutoff_upper, self.cutoff.cutoff_lower))

    def forward(self):
        raise NotImplementedError


class GaussianBasis(_RadialBasis):
    """exp(coeff (d - offset_k)^2) * cutoff(d) with offsets =
    linspace(lower, upper, num_rbf) and coeff = -0.5 / spacing^2.

    Buffers (or parameters when trainable) ``offset`` [K] and ``coeff`` (0-dim)
    carry the reference's state_dict names."""

    def __init__(self, cutoff: Union[int, float, _Cutoff], num_rbf: int = 50,
                 trainable: bool = False):
        super().__init__()
        if isinstance(cutoff, (float, int)):
            self.cutoff = IdentityCutoff(0, cutoff)
        elif isinstance(cutoff, _Cutoff):
            self.cutoff = cutoff
        else:
            raise TypeError(
                "Supplied cutoff {} is neither a number nor a _Cutoff instance.".format(cutoff))
        self.check_cutoff()
        self.num_rbf = num_rbf
        self.trainable = trainable
        offset, coeff = self._initial_params()
        if trainable:
            self.register_parameter("coeff", nn.Parameter(coeff))
            self.register_parameter("offset", nn.Parameter(offset))
        else:
            self.register_buffer("coeff", coeff)
            self.register_buffer("offset", offset)

    def _initial_params(self):
        offset = torch.linspace(self.cutoff.cutoff_lower, self.cutoff.cutoff_upper,
                                self.num_rbf)
        coeff = -0.5 / (offset[1] - offset[0]) ** 2
        return offset, coeff

    def reset_parameters(self):
        offset, coeff = self._initial_params()
        self.offset.data.copy_(offset)
        self.coeff.data.copy_(coeff)

    def forward(self, dist: torch.Tensor) -> torch.Tensor:
        dist = dist.unsqueeze(-1)
        return torch.exp(self.coeff * torch.pow(dist - self.offset, 2)) * self.cutoff(dist)

    @classmethod
    def build_pruned_from_mask(cls, cutoff: Union[int, float, _Cutoff],
                               lambda_mask: torch.Tensor, num_rbf: int = 50,
                               trainable: bool = False):
        """Keeps only the offsets the boolean mask selects (gaussian.py:104-153).
        As in the reference, ``num_rbf`` stays the unpruned count; the
        expansion width is ``offset.numel()``."""
        if lambda_mask.numel() != num_rbf:
            raise ValueError(
                f"lambda_filter must have {num_rbf} elements, got {lambda_mask.numel()}")
        obj = cls(cutoff, num_rbf, trainable)
        lambda_mask = lambda_mask.to(torch.bool).to(obj.offset.device)
        offset = obj.offset[lambda_mask].clone()
        del obj.offset
        if trainable:
            obj.offset = nn.Parameter(offset)
        else:
            obj.register_buffer("offset", offset)
        obj.num_rbf = lambda_mask.numel()
        return obj


class ExpNormalBasis(_RadialBasis):
    """C(d) exp(-beta_k (exp(alpha (lower - d)) - mu_k)^2) with
    alpha = 5 / (upper - lower), mu = linspace(exp(lower - upper), 1, K) and
    beta_k = (2 / K (1 - exp(lower - upper)))^-2 (exp_normal.py:56-130; the
    PhysNet basis).  A float cutoff means CosineCutoff(0, cutoff).  ``means``
    and ``betas`` are parameters when trainable (the default), else buffers."""

    def __init__(self, cutoff: Union[int, float, _Cutoff], num_rbf: int = 50,
                 trainable: bool = True):
        super().__init__()
        if isinstance(cutoff, (float, int)):
            self.cutoff = CosineCutoff(0, cutoff)
        elif isinstance(cutoff, _Cutoff):
            self.cutoff = cutoff
        else:
            raise TypeError(
                "Supplied cutoff {} is neither a number nor a _Cutoff instance.".format(cutoff))
        self.check_cutoff()
        self.num_rbf = num_rbf
        self.trainable = trainable
        self.alpha = 5.0 / (self.cutoff.cutoff_upper - self.cutoff.cutoff_lower)
        means, betas = self._initial_params()
        if trainable:
            self.register_parameter("means", nn.Parameter(means))
            self.register_parameter("betas", nn.Parameter(betas))
        else:
            self.register_buffer("means", means)
            self.register_buffer("betas", betas)

    def _initial_params(self):
        start_value = torch.exp(torch.scalar_tensor(
            -self.cutoff.cutoff_upper + self.cutoff.cutoff_lower))
        means = torch.linspace(start_value, 1, self.num_rbf)
        betas = torch.tensor([(2 / self.num_rbf * (1 - start_value)) ** -2] * self.num_rbf)
        return means, betas

    def reset_parameters(self):
        means, betas = self._initial_params()
        self.means.data.copy_(means)
        self.betas.data.copy_(betas)

    def forward(self, dist: torch.Tensor) -> torch.Tensor:
        dist = dist.unsqueeze(-1)
        return self.cutoff(dist) * torch.exp(
            -self.betas * (torch.exp(self.alpha * (-dist + self.cutoff.cutoff_lower))
                           - self.means) ** 2)

    @classmethod
    def build_pruned_from_mask(cls, cutoff: Union[int, float, _Cutoff],
                               lambda_mask: torch.Tensor, num_rbf: int = 50,
                               trainable: bool = True):
        """Keeps only the basis functions the boolean mask selects
        (exp_normal.py:126-178); ``num_rbf`` stays the unpruned count, as in
        the reference, and the expansion width is ``means.numel()``."""
        if lambda_mask.numel() != num_rbf:
            raise ValueError(
                f"lambda_filter must have {num_rbf} elements, got {lambda_mask.numel()}")
        obj = cls(cutoff, num_rbf, trainable)
        lambda_mask = lambda_mask.to(torch.bool).to(obj.means.device)
        means = obj.means[lambda_mask].clone()
        betas = obj.betas[lambda_mask].clone()
        del obj.means
        del obj.betas
        if trainable:
            obj.means = nn.Parameter(means)
            obj.betas = nn.Parameter(betas)
        else:
            obj.register_buffer("means", means)
            obj.register_buffer("betas", betas)
        obj.num_rbf = lambda_mask.numel()
        return obj
