"""Activations with kernel support.

The fused kernels evaluate Tanh (the reference default,
mlcg/nn/schnet.py:419) and the shifted softplus softplus(x) - ln 2, which the
reference does not define; it is defined here with torch's softplus
(beta = 1, threshold = 20) so the oracle and the kernels agree.
"""

import math

import torch

ACT_TANH = 0
ACT_SSP = 1


class ShiftedSoftplus(torch.nn.Module):
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return torch.nn.functional.softplus(x) - math.log(2.0)


def activation_id(module: torch.nn.Module):
    """Kernel id of an activation module, or None if it has no kernel."""
    if isinstance(module, torch.nn.Tanh):
        return ACT_TANH
    if isinstance(module, ShiftedSoftplus):
        return ACT_SSP
    return None


def act_value(z: torch.Tensor, act: int) -> torch.Tensor:
    if act == ACT_TANH:
        return torch.tanh(z)
    return torch.nn.functional.softplus(z) - math.log(2.0)


def act_derivs(z: torch.Tensor, s: torch.Tensor, act: int):
    """(act'(z), act''(z)) given z and s = act(z)."""
    if act == ACT_TANH:
        d1 = 1.0 - s * s
        return d1, -2.0 * s * d1
    sg = torch.sigmoid(z)
    return sg, sg * (1.0 - sg)
