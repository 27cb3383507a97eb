"""Minimal AtomicData container and collation.

Mirrors the field contract of mlcg's ``AtomicData`` (mlcg/data/atomic_data.py:
21-103) without the PyG ``Data`` dependency: attribute and item access,
``key in data``, an ``out`` dict for model outputs, a ``neighbor_list`` dict,
and collation that offsets every ``*index*`` tensor by the running node
count and ``mapping_batch`` by the frame count (``__inc__``, lines 96-103).
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional

import torch

from ._keys import (
    ATOM_TYPE_KEY,
    BATCH_KEY,
    ENERGY_KEY,
    FORCE_KEY,
    MASS_KEY,
    N_ATOMS_KEY,
    NEIGHBOR_LIST_KEY,
    POSITIONS_KEY,
    VELOCITY_KEY,
    validate_keys,
)


class AtomicData:
    def __init__(self, **kwargs: Any):
        validate_keys(kwargs.keys())
        object.__setattr__(self, "_store", {})
        object.__setattr__(self, "out", {})
        for k, v in kwargs.items():
            self._store[k] = v
        if NEIGHBOR_LIST_KEY not in self._store:
            self._store[NEIGHBOR_LIST_KEY] = {}
        if N_ATOMS_KEY in self and POSITIONS_KEY in self:
            assert int(torch.as_tensor(self.n_atoms).sum()) == self.pos.shape[0], (
                "number of atoms and number of positions differ")
            assert self.pos.shape[1] == 3
        if MASS_KEY in self and POSITIONS_KEY in self:
            assert len(self.masses) == self.pos.shape[0]
        for key in (FORCE_KEY, VELOCITY_KEY):
            if key in self and self[key] is not None:
                assert self[key].shape == self.pos.shape
                assert self[key].dtype == self.pos.dtype

    # attribute / item access -------------------------------------------------
    def __getattr__(self, name: str) -> Any:
        # called only when the normal lookup fails; `_store` is an instance
        # attribute, so reading it here does not recurse (except before it
        # exists, while an instance is being copied or unpickled).  Plain
        # attribute reads also keep the access traceable by torch.compile.
        if name == "_store":
            raise AttributeError(name)
        store = self._store
        if name in store:
            return store[name]
        raise AttributeError(name)

    def __setattr__(self, name: str, value: Any) -> None:
        if name == "out":
            object.__setattr__(self, "out", value)
        else:
            self._store[name] = value

    def __getitem__(self, key: str) -> Any:
        return self._store[key]

    def __setitem__(self, key: str, value: Any) -> None:
        self._store[key] = value

    def __contains__(self, key: str) -> bool:
        return key in self._store and self._store[key] is not None

    def keys(self) -> List[str]:
        return list(self._store.keys())

    @property
    def num_nodes(self) -> int:
        return self.pos.shape[0]

    @property
    def num_graphs(self) -> int:
        if BATCH_KEY in self and self.batch.numel() > 0:
            return int(self.batch[-1]) + 1
        return 1

    def to(self, device) -> "AtomicData":
        def mv(v):
            if isinstance(v, torch.Tensor):
                return v.to(device)
            if isinstance(v, dict):
                return {k: mv(x) for k, x in v.items()}
            return v

        new = AtomicData.__new__(AtomicData)
        object.__setattr__(new, "_store", {k: mv(v) for k, v in self._store.items()})
        object.__setattr__(new, "out", {})
        return new

    def clone(self) -> "AtomicData":
        def cp(v):
            if isinstance(v, torch.Tensor):
                return v.clone()
            if isinstance(v, dict):
                return {k: cp(x) for k, x in v.items()}
            return v

        new = AtomicData.__new__(AtomicData)
        object.__setattr__(new, "_store", {k: cp(v) for k, v in self._store.items()})
        object.__setattr__(new, "out", {})
        return new

    @staticmethod
    def from_points(pos: torch.Tensor, atom_types: torch.Tensor,
                    masses: Optional[torch.Tensor] = None,
                    neighborlist: Optional[Dict] = None, **kwargs) -> "AtomicData":
        """One frame (AtomicData.from_points, atomic_data.py:154-237, no PBC)."""
        fields = {
            POSITIONS_KEY: pos,
            ATOM_TYPE_KEY: atom_types,
            N_ATOMS_KEY: torch.tensor([pos.shape[0]], dtype=torch.long),
            NEIGHBOR_LIST_KEY: neighborlist or {},
        }
        if masses is not None:
            fields[MASS_KEY] = masses
        fields.update(kwargs)
        return AtomicData(**fields)


def _inc(key: str, num_nodes: int) -> int:
    if "index" in key or "face" in key:
        return num_nodes
    if key == "mapping_batch":
        return 1
    return 0


def collate(frames: List[AtomicData]) -> AtomicData:
    """Concatenate frames into one disjoint batch (PyG collation contract)."""
    if not frames:
        raise ValueError("cannot collate an empty list")
    out: Dict[str, Any] = {}
    node_keys = [k for k in frames[0].keys()
                 if k not in (NEIGHBOR_LIST_KEY, N_ATOMS_KEY, ENERGY_KEY, BATCH_KEY)]
    for k in node_keys:
        vals = [f[k] for f in frames]
        if isinstance(vals[0], torch.Tensor):
            out[k] = torch.cat(vals, dim=0)
        else:
            out[k] = vals
    out[N_ATOMS_KEY] = torch.cat([torch.as_tensor(f.n_atoms).view(-1) for f in frames])
    if ENERGY_KEY in frames[0]:
        out[ENERGY_KEY] = torch.cat([torch.as_tensor(f.energy).view(-1) for f in frames])
    out[BATCH_KEY] = torch.cat([
        torch.full((f.num_nodes,), b, dtype=torch.long) for b, f in enumerate(frames)])
    # neighbour lists: concatenate index_mapping with node offsets
    nls: Dict[str, Dict] = {}
    names = frames[0].neighbor_list.keys()
    for name in names:
        parts, mb = [], []
        offset = 0
        for b, f in enumerate(frames):
            nl = f.neighbor_list[name]
            parts.append(nl["index_mapping"] + offset)
            mb.append(torch.full((nl["index_mapping"].shape[1],), b, dtype=torch.long))
            offset += f.num_nodes
        base = dict(frames[0].neighbor_list[name])
        base["index_mapping"] = torch.cat(parts, dim=1)
        base["mapping_batch"] = torch.cat(mb)
        nls[name] = base
    out[NEIGHBOR_LIST_KEY] = nls
    return AtomicData(**out)
