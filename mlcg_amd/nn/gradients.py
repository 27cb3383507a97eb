"""Output wrappers: SumOut, EnergyOut, GradientsOut (mlcg/nn/gradients.py:7-233).

GradientsOut around a fusable HIP SchNet computes energies and forces in one
fused pass (``SchNet.energy_forces``) instead of an autograd replay; in
training mode the result carries the hand-derived force-matching double
backward.  Around a prior it takes the prior kernel's analytic forces.  Any other model goes through torch.autograd exactly like the
reference (lines 208-228).

Under torch.compile (outside training, float32 positions, a batch with
``n_atoms``) the SchNet and prior passes are the custom operator
``mlcg::direct_energy_forces`` and SumOut's sum ``mlcg::sum_arrays``: their
fake implementations let dynamo trace the whole model as one graph.
"""

from __future__ import annotations

from typing import Any, List, Sequence

import torch

from .. import library, ops
from ..data._keys import ENERGY_KEY, FORCE_KEY


class _SumArrays(torch.autograd.Function):
    """Sum of model outputs (ops.sum_arrays); the gradient reaches every input
    unchanged, as through the adds it replaces."""

    @staticmethod
    def forward(ctx, *xs):
        ctx.n = len(xs)
        return ops.sum_arrays(list(xs))

    @staticmethod
    def backward(ctx, g):
        return tuple(g for _ in range(ctx.n))


class SumOut(torch.nn.Module):
    name: str = "SumOut"

    def __init__(self, models: torch.nn.ModuleDict, targets: List[str] = None):
        super().__init__()
        if targets is None:
            targets = [ENERGY_KEY, FORCE_KEY]
        self.targets = targets
        self.models = models

    def forward(self, data):
        if self._outputs_independent():
            # the models never read data.out[target]: run them, then add their
            # outputs in the loop's order in one launch per target
            for name in self.models.keys():
                data = self.models[name](data)
            for target in self.targets:
                parts = [data.out[name][target] for name in self.models.keys()]
                if ops.sum_arrays_ok(parts):
                    if torch.compiler.is_compiling():
                        data.out[target] = torch.ops.mlcg.sum_arrays(parts)
                    else:
                        data.out[target] = _SumArrays.apply(*parts)
                else:
                    acc = 0.00
                    for p in parts:
                        acc += p
                    data.out[target] = acc
            return data
        for target in self.targets:
            data.out[target] = 0.00
        for name in self.models.keys():
            data = self.models[name](data)
            for target in self.targets:
                data.out[target] += data.out[name][target]
        return data

    def _outputs_independent(self) -> bool:
        """Every model is a GradientsOut that writes only data.out[its name]
        (not one wrapping a SumOut, which writes data.out[target] itself)."""
        return len(self.models) > 0 and all(
            isinstance(m, GradientsOut) and m.name != "SumOut" for m in self.models.values())

    def neighbor_list(self, **kwargs):
        nl = {}
        for _, model in self.models.items():
            nl.update(**model.neighbor_list(**kwargs))
        return nl


class EnergyOut(torch.nn.Module):
    name: str = "EnergyOut"

    def __init__(self, model: torch.nn.Module, targets: List[str] = None):
        super().__init__()
        if targets is None:
            targets = [ENERGY_KEY]
        self.targets = targets
        self.model = model
        self.name = self.model.name

    def forward(self, data):
        data = self.model(data)
        for target in self.targets:
            data.out[target] = data.out[self.name][target]
        return data


class GradientsOut(torch.nn.Module):
    _targets = {FORCE_KEY: ENERGY_KEY}

    def __init__(self, model: torch.nn.Module, targets: str = FORCE_KEY):
        super().__init__()
        self.model = model
        self.name = self.model.name
        self.targets = []
        if isinstance(targets, str):
            self.targets = [targets]
        elif isinstance(targets, Sequence):
            self.targets = list(targets)
        assert any(k in GradientsOut._targets for k in self.targets), (
            f"targets={self.targets} should be any of {GradientsOut._targets}")
        library.register_direct_model(model)

    def __setstate__(self, state):
        super().__setstate__(state)
        # a copied or unpickled wrapper holds a new model object
        library.register_direct_model(self.model)

    def _direct_model(self):
        """The wrapped model when it computes energies and forces in one pass
        on the HIP kernels (a fusable SchNet or a prior), else None."""
        from .prior import _Prior
        from .schnet import SchNet

        m = self.model
        if FORCE_KEY not in self.targets:
            return None
        if isinstance(m, SchNet) and m.fused_spec() is not None:
            return m
        if isinstance(m, _Prior):
            return m
        return None

    def _compiled_route(self, data) -> bool:
        """Whether a traced call goes through mlcg::direct_energy_forces
        (decided from types and tensor metadata only, which dynamo evaluates
        while tracing)."""
        from .prior import _Prior
        from .schnet import SchNet

        return (FORCE_KEY in self.targets and not self.training
                and isinstance(self.model, (SchNet, _Prior)) and "n_atoms" in data
                and "batch" in data and data.pos.dtype == torch.float32
                and data.pos.is_cuda)

    def forward(self, data):
        if torch.compiler.is_compiling() and self._compiled_route(data):
            from .prior import _Prior

            mapping = mapping_batch = None
            if isinstance(self.model, _Prior):
                nl = data.neighbor_list[self.model.name]
                mapping = nl["index_mapping"]
                mapping_batch = nl.get("mapping_batch")
            energy, forces = torch.ops.mlcg.direct_energy_forces(
                data.pos.detach(), data.atom_types, data.batch, data.n_atoms, mapping,
                mapping_batch, id(self.model))
            data.out[self.name] = {ENERGY_KEY: energy, FORCE_KEY: forces}
            data.pos = data.pos.detach()
            return data
        direct = self._direct_model()
        if direct is not None:
            energy, forces = direct.energy_forces(data, create_graph=self.training)
            data.out[self.name] = {ENERGY_KEY: energy, FORCE_KEY: forces}
            data.pos = data.pos.detach()
            return data
        data.pos.requires_grad_(True)
        data = self.model(data)
        if FORCE_KEY in self.targets:
            y = data.out[ENERGY_KEY] if self.name == "SumOut" else data.out[self.name][ENERGY_KEY]
            dy_dr = torch.autograd.grad(y.sum(), data.pos, create_graph=self.training)[0]
            if self.name == "SumOut":
                data.out[FORCE_KEY] = -dy_dr
            else:
                data.out[self.name][FORCE_KEY] = -dy_dr
        data.pos = data.pos.detach()
        return data

    def neighbor_list(self, **kwargs: Any):
        return self.model.neighbor_list(**kwargs)
