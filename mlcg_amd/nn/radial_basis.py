"""Gaussian radial basis (mlcg/nn/radial_basis/gaussian.py:9-102, base.py:4-41)."""

from typing import Union

import torch
from torch import nn

from .cutoff import IdentityCutoff, _Cutoff


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
