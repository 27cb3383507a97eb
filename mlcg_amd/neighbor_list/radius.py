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
from .._lib import require_device


def radius_graph(x: torch.Tensor, r: float, batch: Optional[torch.Tensor] = None,
                 loop: bool = False, max_num_neighbors: int = 32,
                 flow: str = "target_to_source") -> torch.Tensor:
    """[2, E] int64 edge list; torch_cluster.radius_graph call signature.

    With flow="target_to_source" row 0 is the centre (as mlcg calls it,
    torch_impl.py:216-224); "source_to_target" swaps the rows."""
    xm = x.detach() if x.dtype == torch.float64 else x.detach().float()
    g = ops.radius_graph(xm, r, batch=batch, loop=loop, max_num_neighbors=max_num_neighbors)
    ei = g.edge_index
    if flow == "source_to_target":
        ei = ei.flip(0)
    elif flow != "target_to_source":
        raise ValueError(f"unknown flow {flow!r}")
    return ei


exclusion_pair_to_ptr = ops.exclusion_pair_to_ptr


def radius_cuda(x: torch.Tensor, ptr_x: Optional[torch.Tensor], r: float,
                max_num_neighbors: int, ignore_same_index: bool,
                exclude_pair_xs: Optional[torch.Tensor] = None,
                ptr_exclude_pair_xs: Optional[torch.Tensor] = None):
    """(edge_index [2, E] int64, distance [E]) with the arguments of the
    reference's native operator ``mlcg::radius_cuda`` (radius.cu:197-307):
    frames given by ``ptr_x`` [B+1] (None = one frame), optional exclusion CSR.
    Edges come out in canonical (centre, neighbour) order.  x is float32,
    float64, float16 or bfloat16, the membership test running in x's type as
    in the reference's dispatch (radius.cu:243-250); the distances are in x's
    type (for the 16-bit types with every operation rounded to it, as the
    reference's kernel computes sqrt(dist))."""
    require_device(x)
    _check_2d(x)
    if x.dtype not in _RADIUS_DTYPES:
        raise RuntimeError(
            f"radius_cuda takes float32, float64, float16 or bfloat16 positions, got {x.dtype}")
    n = x.shape[0]
    if ptr_x is None:
        ptr_x = torch.tensor([0, n], dtype=torch.int64, device=x.device)
    require_device(ptr_x)
    ptr_x = ptr_x.to(torch.int64).contiguous()
    if ptr_x.dim() != 1:
        raise RuntimeError("ptr_x must be 1-D")
    nodes = torch.arange(n, device=x.device)
    batch = torch.searchsorted(ptr_x, nodes, right=True) - 1
    g = ops.radius_graph(x.detach(), r, batch=batch, loop=not ignore_same_index,
                         max_num_neighbors=max_num_neighbors, frame_ptr=ptr_x,
                         exclude_pair_xs=exclude_pair_xs,
                         ptr_exclude_pair_xs=ptr_exclude_pair_xs)
    ei = g.edge_index
    return ei, _edge_distances(x.detach(), ei)


_RADIUS_DTYPES = (torch.float32, torch.float64, torch.float16, torch.bfloat16)


def _edge_distances(x: torch.Tensor, ei: torch.Tensor) -> torch.Tensor:
    """|x_j - x_i| over the edges (i = ei[0], j = ei[1]).  For float16 and
    bfloat16 it is the reference kernel's sequence in x's type, every
    operation rounded (radius.cu:117-124): d = x_j - x_i, d2 = (dx^2 + dy^2) +
    dz^2, sqrt(d2); torch evaluates each such elementwise operation in float
    and rounds it, the c10 arithmetic."""
    if x.dtype in (torch.float16, torch.bfloat16) and x.shape[1] == 3:
        d = x[ei[1]] - x[ei[0]]
        sq = d * d
        return torch.sqrt((sq[:, 0] + sq[:, 1]) + sq[:, 2])
    return (x[ei[0]] - x[ei[1]]).norm(dim=1)


def _check_2d(x: torch.Tensor) -> None:
    if x.dim() != 2:
        raise RuntimeError(f"x must be [N, D], got {tuple(x.shape)}")


def radius_distance_fn(x: torch.Tensor, r: float, batch: Optional[torch.Tensor] = None,
                       loop: bool = False, max_num_neighbors: int = 32,
                       batch_size: Optional[int] = None,
                       exclude_pair_indices: Optional[torch.Tensor] = None):
    """(edge_index [2, E], distance [E]) like radius.py:52-88, including the
    optional exclusion pair list [2, M] (converted by exclusion_pair_to_ptr,
    radius.py:77-84)."""
    if x.numel() == 0:
        return (torch.empty(2, 0, dtype=torch.long, device=x.device),
                torch.empty(0, dtype=x.dtype, device=x.device))
    exs = eptr = None
    if exclude_pair_indices is not None:
        exs, eptr = ops.exclusion_pair_to_ptr(exclude_pair_indices, x.size(0))
    # membership is decided in x's own type (the reference's scalar-type
    # dispatch, radius.cu:243-250); the distances are computed in x's dtype
    # so fp64 gradchecks stay exact
    xm = x.detach() if x.dtype in _RADIUS_DTYPES else x.detach().float()
    g = ops.radius_graph(xm, r, batch=batch, loop=loop,
                         max_num_neighbors=max_num_neighbors, n_frames=batch_size,
                         exclude_pair_xs=exs, ptr_exclude_pair_xs=eptr)
    ei = g.edge_index
    return ei, _edge_distances(x.detach(), ei)


class RadiusDistanceAGF(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, r, batch, loop, max_num_neighbors, batch_size,
                exclude_pair_indices=None):
        edge_index, distance = radius_distance_fn(x, r, batch, loop, max_num_neighbors,
                                                  batch_size, exclude_pair_indices)
        ctx.save_for_backward(x, distance, edge_index)
        ctx.mark_non_differentiable(edge_index)
        return distance, edge_index

    @staticmethod
    def backward(ctx, grad_d, grad_ei):
        x, distance, edge_index = ctx.saved_tensors
        return (RadiusDistanceAGB.apply(x, distance, grad_d, edge_index),) + (None,) * 6


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
                    batch_size: Optional[int] = None,
                    exclude_pair_indices: Optional[torch.Tensor] = None,
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
    """(distance [E], edge_index [2, E]) with autograd on the distances
    (radius.py:187-199)."""
    return RadiusDistanceAGF.apply(x, r, batch, loop, max_num_neighbors, batch_size,
                                   exclude_pair_indices)
