"""MLP and Xavier initialisation (mlcg/nn/mlp.py:7-58, _module_init.py:4-28)."""

from typing import List

import torch


def init_xavier_uniform(module: torch.nn.Module, zero_bias: bool = True) -> None:
    """In-place Xavier-uniform weights and zero bias for torch.nn.Linear."""
    if isinstance(module, torch.nn.Linear):
        torch.nn.init.xavier_uniform_(module.weight)
        if module.bias is not None and zero_bias:
            torch.nn.init.constant_(module.bias, 0.0)


class MLP(torch.nn.Module):
    """[Linear(bias) -> act]* -> Linear(bias=last_bias); the activation modules
    sit at the odd indices of ``layers`` so state_dict keys match the
    reference (``layers.0.weight``, ``layers.2.weight`` ...)."""

    def __init__(self, layer_widths: List[int] = None,
                 activation_func: torch.nn.Module = torch.nn.Tanh(), last_bias: bool = True):
        super().__init__()
        if layer_widths is None:
            layer_widths = [10, 10, 1]
        layers = []
        for w_in, w_out in zip(layer_widths[:-2], layer_widths[1:-1]):
            layers.append(torch.nn.Linear(w_in, w_out, bias=True))
            layers.append(activation_func)
        layers.append(torch.nn.Linear(layer_widths[-2], layer_widths[-1], bias=last_bias))
        self.layers = torch.nn.Sequential(*layers)
        self.reset_parameters()

    def reset_parameters(self):
        for layer in self.layers:
            init_xavier_uniform(layer)

    def forward(self, x, data=None):
        return self.layers(x)

    def linears(self) -> List[torch.nn.Linear]:
        return [m for m in self.layers if isinstance(m, torch.nn.Linear)]

    def activations(self) -> List[torch.nn.Module]:
        return [m for m in self.layers if not isinstance(m, torch.nn.Linear)]
