"""``radius_distance`` / ``radius_graph`` Python API of the reference's native
radius operator (src/opt_radius/mlcg_opt_radius/radius.py:52-199) on the
gfx950 kernel.

The autograd of the distances follows the reference's hand-written first and
second derivatives (RadiusDistanceAGF/AGB, radius.py:91-158).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import ops


def radius_graph(x: torch.Tensor, r: float, batch: Optional[torch.Tensor] = None,
                 loop: bool = False, max_num_neighbors: int = 32,
                 flow: str = "target_to_source") -> torch.Tensor:
    """[2, E] int64 edge list; torch_cluster.radius_graph call signature.

    With flow="target_to_source" row 0 is the centre (as mlcg calls it,
    torch_impl.py:216-224); "source_to_target" swaps the rows."""
    g = ops.radius_graph(x.detach().float(), r, batch=batch, loop=loop,
                         max_num_neighbors=max_num_neighbors)
    ei = g.edge_index
    if flow == "source_to_target":
        ei = ei.flip(0)
    elif flow != "target_to_source":
        raise ValueError(f"unknown flow {flow!r}")
    return ei


def radius_distance_fn(x: torch.Tensor, r: float, batch: Optional[torch.Tensor] = None,
                       loop: bool = False, max_num_neighbors: int = 32,
                       batch_size: Optional[int] = None):
    """(edge_index [2, E], distance [E]) like radius.py:52-88."""
    # membership is decided in fp32 (the kernel's arithmetic); the distances
    # themselves are computed in x's dtype so fp64 gradchecks stay exact
    g = ops.radius_graph(x.detach().float(), r, batch=batch, loop=loop,
                         max_num_neighbors=max_num_neighbors, n_frames=batch_size)
    ei = g.edge_index
    d = (x.detach()[ei[0]] - x.detach()[ei[1]]).norm(dim=1)
    return ei, d


class RadiusDistanceAGF(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, r, batch, loop, max_num_neighbors, batch_size):
        edge_index, distance = radius_distance_fn(x, r, batch, loop, max_num_neighbors,
                                                  batch_size)
        ctx.save_for_backward(x, distance, edge_index)
        ctx.mark_non_differentiable(edge_index)
        return distance, edge_index

    @staticmethod
    def backward(ctx, grad_d, grad_ei):
        x, distance, edge_index = ctx.saved_tensors
        return (RadiusDistanceAGB.apply(x, distance, grad_d, edge_index),) + (None,) * 5


class RadiusDistanceAGB(torch.autograd.Function):
    """d(distance)/dx and its derivative (radius.py:123-158)."""

    @staticmethod
    def forward(ctx, x, distance, grad_d, edge_index):
        ei, ej = edge_index[0], edge_index[1]
        diff = x[ei] - x[ej]
        scaling = (grad_d / distance).unsqueeze(-1)
        gx = torch.zeros_like(x)
        gx.index_add_(0, ei, scaling * diff)
        gx.index_add_(0, ej, -scaling * diff)
        ctx.save_for_backward(edge_index, diff, scaling, grad_d, distance)
        return gx

    @staticmethod
    def backward(ctx, gout):
        edge_index, diff, scaling, grad_d, distance = ctx.saved_tensors
        ei, ej = edge_index[0], edge_index[1]
        dg = gout[ei] - gout[ej]
        dgd = (dg * diff).sum(dim=1)
        term = scaling * dg
        gx = torch.zeros_like(gout)
        gx.index_add_(0, ei, term)
        gx.index_add_(0, ej, -term)
        return gx, -grad_d * dgd / distance ** 2, dgd / distance, None


def radius_distance(x: torch.Tensor, r: float, batch: Optional[torch.Tensor] = None,
                    loop: bool = False, max_num_neighbors: int = 32,
                    batch_size: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(distance [E], edge_index [2, E]) with autograd on the distances."""
    return RadiusDistanceAGF.apply(x, r, batch, loop, max_num_neighbors, batch_size)
