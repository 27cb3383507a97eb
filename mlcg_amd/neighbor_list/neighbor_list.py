"""Neighbour-list dictionaries (mlcg/neighbor_list/neighbor_list.py:27-202).

``atomic_data2neighbor_list`` keeps the reference's backend switch
(``nls_distance_method``, lines 58-72): "torch", "custom_kernel" and "hip"
all resolve to the gfx950 radius graph (``mlcg_amd.ops.radius_graph``); the
NVIDIA nvalchemi backends are not available in this build.
"""

from __future__ import annotations

from typing import Dict, Mapping, Optional

import torch

from .. import ops

_BACKENDS = ("torch", "custom_kernel", "hip")


def hip_neighbor_list(data, rcut: float, self_interaction: bool = False,
                      max_num_neighbors: int = 1000):
    """(idx_i, idx_j, cell_shifts, mask) in the backend signature of
    neighbor_list.py:73-78 (torch_neighbor_list for non-periodic data)."""
    n = data.pos.shape[0]
    batch = data.batch if "batch" in data else torch.zeros(
        n, dtype=torch.long, device=data.pos.device)
    n_frames = int(data.n_atoms.numel()) if "n_atoms" in data else None
    g = ops.radius_graph(data.pos.detach(), rcut, batch=batch, loop=self_interaction,
                         max_num_neighbors=max_num_neighbors, n_frames=n_frames)
    ei = g.edge_index
    cell_shifts = torch.zeros((ei.shape[1], 3), dtype=data.pos.dtype, device=data.pos.device)
    return ei[0], ei[1], cell_shifts, ei[0] != ei[1]


def atomic_data2neighbor_list(data, rcut: float, self_interaction: bool = False,
                              max_num_neighbors: int = 1000,
                              nls_distance_method: str = "torch") -> Dict:
    rcut = float(rcut)
    if nls_distance_method not in _BACKENDS:
        raise ValueError(
            f"Method {nls_distance_method} not supported for nls-distance computation ")
    if "pbc" in data and bool(torch.as_tensor(data.pbc).any()):
        raise NotImplementedError("periodic systems are not supported by the HIP radius graph")
    idx_i, idx_j, cell_shifts, _ = hip_neighbor_list(
        data, rcut, self_interaction=self_interaction, max_num_neighbors=max_num_neighbors)
    mapping = torch.stack([idx_i, idx_j], dim=0)
    order = mapping.shape[0]
    batch = data.batch if "batch" in data else torch.zeros(
        data.pos.shape[0], dtype=torch.long, device=data.pos.device)
    # every edge stays inside its frame by construction (the reference asserts
    # it, neighbor_list.py:89-91)
    mapping_batch = batch[mapping[0]]
    return make_neighbor_list(tag=f"nonbounded rc:{rcut} order:{order}", order=order,
                              index_mapping=mapping, mapping_batch=mapping_batch,
                              cell_shifts=cell_shifts, rcut=rcut,
                              self_interaction=self_interaction)


def make_neighbor_list(tag: str, order: int, index_mapping: torch.Tensor,
                       mapping_batch: Optional[torch.Tensor] = None,
                       cell_shifts: Optional[torch.Tensor] = None, rcut: Optional[float] = None,
                       self_interaction: Optional[bool] = None) -> Dict:
    """neighbor_list.py:105-163."""
    if index_mapping.shape[0] != order:
        raise RuntimeError(
            f"index_mapping shape does not match the order:{index_mapping.shape[0]} != {order}")
    if mapping_batch is None:
        mapping_batch = torch.zeros((index_mapping.shape[1],), dtype=torch.long,
                                    device=index_mapping.device)
    return dict(tag=tag, order=order,
                index_mapping=torch.as_tensor(index_mapping, dtype=torch.long),
                cell_shifts=cell_shifts, rcut=rcut, self_interaction=self_interaction,
                mapping_batch=mapping_batch)


class _EmptyField:
    pass


def validate_neighborlist(inp) -> bool:
    """neighbor_list.py:170-202."""
    validator = {"tag": [str], "order": [int], "index_mapping": [torch.Tensor],
                 "cell_shifts": [torch.Tensor], "rcut": [float], "self_interaction": [bool]}
    if not isinstance(inp, Mapping):
        return False
    return all(any(isinstance(inp.get(k, _EmptyField()), t) for t in types)
               for k, types in validator.items())
