"""torch.library registrations of the reference's native operators.

The reference registers ``mlcg::radius_cuda`` (src/opt_radius/mlcg_opt_radius/
radius.cu:313-314) and ``mlcg::exclusion_pair_to_ptr`` (exclusion_pairs.cpp:
64-65) as TorchScript operators.  The same two names are registered here as
``torch.library.custom_op``s backed by the gfx950 kernels, with fake
(meta) implementations, so that code calling ``torch.ops.mlcg.radius_cuda``
runs unchanged and ``torch.compile`` can trace through the calls (the edge
count is data-dependent: the fake implementation returns an unbacked size).

If another library already defines the ``mlcg`` operators (the reference's own
CUDA extension), nothing is registered.

Two operators of this library's own (no counterpart in the reference) make the
fused model visible to ``torch.compile`` (the reference's simulation compiles
its model, simulation/base.py:447-489):

  ``mlcg::direct_energy_forces``  energies [B] and forces [N, 3] of one model
      wrapped by GradientsOut (a SchNet or a prior), found by the id of the
      module, which GradientsOut registers;
  ``mlcg::sum_arrays``  SumOut's sum of its models' outputs (mlcg_sum_arrays),
      with the gradient passed to every input.

Their fake implementations give the output shapes, so a compiled model
holding them traces without graph breaks (``fullgraph=True``) and
``mode="reduce-overhead"`` can capture the whole call.
"""

from __future__ import annotations

import weakref
from typing import List, Optional, Tuple

import torch

REGISTERED = False
MODEL_OPS_REGISTERED = False

# modules reachable from mlcg::direct_energy_forces, by id(module)
_DIRECT_MODELS: "weakref.WeakValueDictionary[int, torch.nn.Module]" = weakref.WeakValueDictionary()


def register_direct_model(module: torch.nn.Module) -> None:
    """Makes `module` reachable from mlcg::direct_energy_forces as
    id(module) (GradientsOut registers the model it wraps, also when it is
    copied or unpickled)."""
    _DIRECT_MODELS[id(module)] = module


class _DirectData:
    """The fields of a batch that the energy/force passes read: positions,
    types, frame index and sizes, and the prior's interaction list."""

    def __init__(self, pos, atom_types, batch, n_atoms, name, mapping, mapping_batch):
        self.pos = pos
        self.atom_types = atom_types
        self.batch = batch
        self.n_atoms = n_atoms
        nl = {}
        if mapping is not None:
            nl["index_mapping"] = mapping
            if mapping_batch is not None:
                nl["mapping_batch"] = mapping_batch
        self.neighbor_list = {name: nl}
        self.out = {}

    def __contains__(self, key: str) -> bool:
        return key in ("pos", "atom_types", "batch", "n_atoms", "neighbor_list")


_AUTOGRAD_KEYS = tuple(getattr(torch._C.DispatchKey, k) for k in (
    "AutogradFunctionality", "AutogradOther", "AutogradCPU", "AutogradCUDA",
    "AutogradNestedTensor") if hasattr(torch._C.DispatchKey, k))


def _energy_forces(model: torch.nn.Module, data: _DirectData):
    """(E, F) of a SchNet or a prior: the fused pass when the model has one,
    else the model's forward and the position gradient, as GradientsOut
    computes them."""
    from .data._keys import ENERGY_KEY
    from .nn.prior import _Prior
    from .nn.schnet import SchNet

    if isinstance(model, _Prior) or (isinstance(model, SchNet) and model.fused_spec() is not None):
        return model.energy_forces(data, create_graph=False)
    # an operator's implementation runs with the autograd dispatch keys
    # excluded; the module path takes its position gradient from autograd, so
    # they are allowed again for this computation
    exclude = torch._C._dispatch_tls_local_exclude_set()
    for key in _AUTOGRAD_KEYS:
        exclude = exclude.remove(key)
    with torch._C._ForceDispatchKeyGuard(torch._C._dispatch_tls_local_include_set(), exclude), \
            torch.enable_grad():
        pos = data.pos.detach().requires_grad_(True)
        data.pos = pos
        data = model(data)
        E = data.out[model.name][ENERGY_KEY]
        (dE,) = torch.autograd.grad(E.sum(), pos)
    return E.detach(), -dE


def register_model_ops() -> None:
    """Registers mlcg::direct_energy_forces and mlcg::sum_arrays (once)."""
    global MODEL_OPS_REGISTERED
    if MODEL_OPS_REGISTERED:
        return

    @torch.library.custom_op("mlcg::direct_energy_forces", mutates_args=())
    def direct_energy_forces_op(pos: torch.Tensor, atom_types: torch.Tensor,
                                batch: torch.Tensor, n_atoms: torch.Tensor,
                                mapping: Optional[torch.Tensor],
                                mapping_batch: Optional[torch.Tensor],
                                model_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """(E [n_frames], F [N, 3]) of the registered model id(model) ==
        model_id on the batch (pos, atom_types, batch, n_atoms) and, for a
        prior, its interaction list (mapping, mapping_batch)."""
        model = _DIRECT_MODELS.get(model_id)
        if model is None:
            raise RuntimeError("mlcg::direct_energy_forces: no model registered under this id "
                               "(GradientsOut registers the model it wraps)")
        E, F = _energy_forces(model, _DirectData(pos, atom_types, batch, n_atoms, model.name,
                                                 mapping, mapping_batch))
        return E.contiguous(), F.contiguous()

    @direct_energy_forces_op.register_fake
    def _direct_fake(pos, atom_types, batch, n_atoms, mapping, mapping_batch, model_id):
        if pos.dim() != 2 or pos.shape[1] != 3:
            raise RuntimeError(f"pos must be [N, 3], got {tuple(pos.shape)}")
        return pos.new_empty((n_atoms.shape[0],)), pos.new_empty(pos.shape)

    @torch.library.custom_op("mlcg::sum_arrays", mutates_args=())
    def sum_arrays_op(xs: List[torch.Tensor]) -> torch.Tensor:
        """((0 + xs[0]) + xs[1]) + ... in one launch (1..8 contiguous float32
        tensors of one shape on one GPU)."""
        from . import ops

        return ops.sum_arrays(list(xs))

    @sum_arrays_op.register_fake
    def _sum_fake(xs):
        return torch.empty_like(xs[0])

    def _sum_setup(ctx, inputs, output):
        ctx.n = len(inputs[0])

    def _sum_backward(ctx, g):
        return [g] * ctx.n

    sum_arrays_op.register_autograd(_sum_backward, setup_context=_sum_setup)
    MODEL_OPS_REGISTERED = True


def _already_defined(name: str) -> bool:
    try:
        getattr(torch.ops.mlcg, name)
        return True
    except (AttributeError, RuntimeError):
        return False


def register() -> bool:
    """Registers the two operators (once); returns whether they are ours."""
    global REGISTERED
    if REGISTERED:
        return True
    if _already_defined("radius_cuda") or _already_defined("exclusion_pair_to_ptr"):
        return False

    @torch.library.custom_op("mlcg::radius_cuda", mutates_args=())
    def radius_cuda_op(x: torch.Tensor, ptr_x: Optional[torch.Tensor], r: float,
                       max_num_neighbors: int, ignore_same_index: bool,
                       exclude_pair_xs: Optional[torch.Tensor] = None,
                       ptr_exclude_pair_xs: Optional[torch.Tensor] = None
                       ) -> Tuple[torch.Tensor, torch.Tensor]:
        """(edge_index [2, E] int64, distance [E]) of the frames of x
        (radius.cu:197-307); see mlcg_amd.neighbor_list.radius.radius_cuda."""
        from .neighbor_list.radius import radius_cuda

        ei, d = radius_cuda(x, ptr_x, r, max_num_neighbors, ignore_same_index,
                            exclude_pair_xs, ptr_exclude_pair_xs)
        return ei.contiguous(), d.contiguous()

    @radius_cuda_op.register_fake
    def _radius_cuda_fake(x, ptr_x, r, max_num_neighbors, ignore_same_index,
                          exclude_pair_xs=None, ptr_exclude_pair_xs=None):
        if x.dim() != 2:
            raise RuntimeError(f"x must be [N, D], got {tuple(x.shape)}")
        n_edges = torch.library.get_ctx().new_dynamic_size()
        return (x.new_empty((2, n_edges), dtype=torch.int64), x.new_empty((n_edges,)))

    @torch.library.custom_op("mlcg::exclusion_pair_to_ptr", mutates_args=())
    def exclusion_pair_to_ptr_op(exc_pair_index: torch.Tensor,
                                 num_nodes: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """(pair_xs [M], y_ptr [num_nodes + 1]) (exclusion_pairs.cpp:7-62)."""
        from . import ops

        xs, ptr = ops.exclusion_pair_to_ptr(exc_pair_index, num_nodes)
        return xs.contiguous(), ptr.contiguous()

    @exclusion_pair_to_ptr_op.register_fake
    def _exclusion_fake(exc_pair_index, num_nodes):
        if exc_pair_index.dim() != 2 or exc_pair_index.shape[0] != 2:
            raise RuntimeError("exc_pair_index must be [2, M]")
        return (exc_pair_index.new_empty((exc_pair_index.shape[1],), dtype=torch.int64),
                exc_pair_index.new_empty((num_nodes + 1,), dtype=torch.int64))

    REGISTERED = True
    return True
