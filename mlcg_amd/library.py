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
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

REGISTERED = False


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
