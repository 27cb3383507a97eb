"""Cutoff envelopes (mlcg/nn/cutoff.py:8-153).

The module forwards are the reference formulas in torch ops (used by the
standalone CFConv/GaussianBasis API); inside the fused SchNet path the same
envelopes, and their distance derivatives, are evaluated in the filter kernel
(mlcg_amd/csrc/common.h: mlcg_cutoff).
"""

import math

import numpy as np
import torch
import torch.nn as nn


class _Cutoff(nn.Module):
    """Abstract cutoff (cutoff.py:8-25)."""

    kind_id = -1

    def __init__(self):
        super().__init__()
        self.cutoff_lower = None
        self.cutoff_upper = None

    def check_cutoff(self):
        if self.cutoff_upper < self.cutoff_lower:
            raise ValueError(
                "Upper cutoff {} is less than lower cutoff {}".format(
                    self.cutoff_upper, self.cutoff_lower))

    def forward(self):
        raise NotImplementedError


class IdentityCutoff(_Cutoff):
    """Envelope equal to one everywhere (cutoff.py:40-72)."""

    kind_id = 0

    def __init__(self, cutoff_lower: float = 0, cutoff_upper: float = np.inf):
        super().__init__()
        self.cutoff_lower = cutoff_lower
        self.cutoff_upper = cutoff_upper
        self.check_cutoff()

    def forward(self, distances: torch.Tensor) -> torch.Tensor:
        return torch.ones_like(distances)


class CosineCutoff(_Cutoff):
    """Cosine envelope on [lower, upper] (cutoff.py:75-153)."""

    kind_id = 1

    def __init__(self, cutoff_lower: float = 0.0, cutoff_upper: float = 5.0):
        super().__init__()
        self.cutoff_lower = cutoff_lower
        self.cutoff_upper = cutoff_upper
        self.check_cutoff()

    def forward(self, distances: torch.Tensor) -> torch.Tensor:
        if self.cutoff_lower > 0:
            cutoffs = 0.5 * (torch.cos(math.pi * (
                2 * (distances - self.cutoff_lower)
                / (self.cutoff_upper - self.cutoff_lower) + 1.0)) + 1.0)
            cutoffs = cutoffs * (distances < self.cutoff_upper).to(distances.dtype)
            cutoffs = cutoffs * (distances > self.cutoff_lower).to(distances.dtype)
            return cutoffs
        cutoffs = 0.5 * (torch.cos(distances * math.pi / self.cutoff_upper) + 1.0)
        return cutoffs * (distances < self.cutoff_upper).to(distances.dtype)
