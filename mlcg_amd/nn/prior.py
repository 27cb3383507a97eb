"""Prior energy modules on the HIP prior kernels (mlcg/nn/prior/).

Same constructors, parameter tables (buffers ``x_0``/``k``, ``k1s``/``k2s``/
``v_0``, ``sigma`` indexed by bead types), names ("bonds", "angles",
"dihedrals", "repulsion") and ``forward(data) -> data.out[name]["energy"]``
contract as the reference:

  Harmonic / HarmonicBonds / HarmonicAngles   prior/harmonic.py:22-298
  FourierSeries / Dihedral                    prior/fourier_series.py:16-198,446-483
  Repulsion                                   prior/repulsion.py:14-238

Energies and analytic forces come from one kernel per prior
(``mlcg_prior_terms``) plus a deterministic per-bead force reduction; the
interaction -> bead index structures are built once per neighbour list and
cached.  ``energy_forces`` gives both at once (what GradientsOut uses); the
plain ``forward`` result is differentiable with respect to ``data.pos`` for
callers that take the position gradient themselves.  The priors hold
buffers only, so no parameter gradients exist.
"""

from __future__ import annotations

from typing import Dict, Final, Optional, Tuple

import torch

from .. import ops
from .._lib import require_device
from ..data._keys import ENERGY_KEY


class _PriorEnergy(torch.autograd.Function):
    """E [B] of one prior; backward gives dE/dpos from the kernel's forces."""

    @staticmethod
    def forward(ctx, pos, kind, n_degs, graph, params, batch):
        E, F = ops.prior_energy_forces(kind, n_degs, pos.detach(), graph, params)
        ctx.save_for_backward(F, batch)
        return E

    @staticmethod
    def backward(ctx, gE):
        F, batch = ctx.saved_tensors
        gpos = -(gE.index_select(0, batch).unsqueeze(1) * F)
        return gpos, None, None, None, None, None


def _pos_for_kernels(pos: torch.Tensor) -> torch.Tensor:
    """float64 positions stay double (a model moved to double, the reference's
    dtype="double" simulations); anything else runs in float32."""
    return pos if pos.dtype == torch.float64 else pos.float()


def _n_frames(data) -> int:
    if "n_atoms" in data:
        return int(data.n_atoms.numel())
    if "batch" in data and data.batch.numel() > 0:
        return int(data.batch[-1]) + 1
    return 1


class _Prior(torch.nn.Module):
    """Base class (prior/base.py:80-141) with the kernel plumbing."""

    name: str = ""
    kind: int = -1
    n_degs: int = 0

    def __init__(self) -> None:
        super().__init__()
        self._graph_key = None
        self._graph: Optional[ops.PriorGraph] = None
        self._pcache = None

    def _params(self, data) -> torch.Tensor:
        """param_matrix(data), reused while the interaction list, the atom
        types and the parameter tables are the same tensors at the same
        versions: a simulation evaluates the per-interaction lookup once
        instead of every step (and a captured step holds no lookup kernels).
        The cache keeps references to the tensors it was built from, so their
        memory cannot be reused by other tensors while it is valid."""
        mapping = data.neighbor_list[self.name]["index_mapping"]
        types = data.atom_types
        bufs = tuple(self.buffers())
        if any(b.requires_grad for b in bufs):
            return self.param_matrix(data)
        key = (mapping._version, types._version, tuple(b._version for b in bufs),
               tuple(b.data_ptr() for b in bufs))
        c = getattr(self, "_pcache", None)
        if c is not None and c[0] is mapping and c[1] is types and c[2] == key:
            return c[3]
        m = self.param_matrix(data).contiguous()
        self._pcache = (mapping, types, key, m)
        return m

    def data2parameters(self, data) -> Dict[str, torch.Tensor]:
        raise NotImplementedError

    def param_matrix(self, data) -> torch.Tensor:
        """[M, n_params] per-interaction parameters in the kernel's layout."""
        raise NotImplementedError

    def prior_graph(self, data) -> ops.PriorGraph:
        nl = data.neighbor_list[self.name]
        mapping = nl["index_mapping"]
        mb = nl.get("mapping_batch")
        key = (mapping.data_ptr(), tuple(mapping.shape), mapping._version,
               None if mb is None else (mb.data_ptr(), mb._version), data.pos.shape[0],
               _n_frames(data))
        if key != self._graph_key:
            self._graph = ops.prior_graph(mapping, mb, data.pos.shape[0], _n_frames(data))
            self._graph_key = key
        return self._graph

    def _batch(self, data) -> torch.Tensor:
        if "batch" in data:
            return data.batch
        return torch.zeros(data.pos.shape[0], dtype=torch.long, device=data.pos.device)

    @torch.compiler.disable  # kernel launches: opaque to torch.compile
    def forward(self, data):
        require_device(data.pos)
        g = self.prior_graph(data)
        E = _PriorEnergy.apply(_pos_for_kernels(data.pos), self.kind, self.n_degs, g,
                               self._params(data), self._batch(data))
        data.out[self.name] = {ENERGY_KEY: E}
        return data

    @torch.compiler.disable
    def energy_forces(self, data, create_graph: bool = False,
                      forces: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """(E [B], F [N, 3]); F is added into `forces` when given."""
        require_device(data.pos)
        g = self.prior_graph(data)
        return ops.prior_energy_forces(self.kind, self.n_degs, _pos_for_kernels(data.pos.detach()), g,
                                       self._params(data), forces=forces)

    def _types(self, data, order):
        mapping = data.neighbor_list[self.name]["index_mapping"]
        return tuple(data.atom_types[mapping[ii]] for ii in range(order))


class Harmonic(_Prior):
    """U = k (x - x0)^2 (+ V0) on a bond length or an angle cosine
    (prior/harmonic.py:22-120)."""

    def __init__(self, statistics: Dict, name: str, order: int) -> None:
        super().__init__()
        keys = torch.tensor(list(statistics.keys()), dtype=torch.long)
        self.allowed_interaction_keys = list(statistics.keys())
        self.name = name
        self.order = order
        unique_types = torch.unique(keys.flatten())
        assert unique_types.min() >= 0
        max_type = int(unique_types.max())
        sizes = tuple(max_type + 1 for _ in range(order))
        x_0 = torch.zeros(sizes)
        k = torch.zeros(sizes)
        for key in statistics.keys():
            x_0[key] = statistics[key]["x_0"]
            k[key] = statistics[key]["k"]
        self.register_buffer("x_0", x_0)
        self.register_buffer("k", k)

    def data2parameters(self, data):
        t = self._types(data, self.order)
        params = {"x0": self.x_0[t].flatten(), "k": self.k[t].flatten()}
        params["V0"] = torch.zeros_like(params["x0"])
        return params

    def param_matrix(self, data):
        p = self.data2parameters(data)
        v0 = p.get("V0")
        if v0 is None:
            v0 = torch.zeros_like(p["x0"])
        return torch.stack([p["x0"].flatten(), p["k"].flatten(), v0.flatten()], dim=1)

    @staticmethod
    def compute(x, x0, k, V0=0):
        return k * (x - x0) ** 2 + V0


class HarmonicBonds(Harmonic):
    name: Final[str] = "bonds"
    _order = 2
    kind = ops.PRIOR_KIND["bonds"]

    def __init__(self, statistics) -> None:
        super().__init__(statistics, HarmonicBonds.name, order=2)


class HarmonicAngles(Harmonic):
    """Harmonic in cos(theta) (prior/harmonic.py:245-298)."""

    name: Final[str] = "angles"
    _order = 3
    kind = ops.PRIOR_KIND["angles"]

    def __init__(self, statistics) -> None:
        super().__init__(statistics, HarmonicAngles.name, order=3)


class FourierSeries(_Prior):
    """V = v0 + sum_n k1_n sin(n t) + k2_n cos(n t)
    (prior/fourier_series.py:16-198)."""

    kind = ops.PRIOR_KIND["dihedrals"]

    def __init__(self, statistics: Dict, name: str = "", n_degs: int = 6,
                 order: int = 4) -> None:
        super().__init__()
        keys = torch.tensor(list(statistics.keys()), dtype=torch.long)
        self.allowed_interaction_keys = list(statistics.keys())
        self.order = order
        self.name = name
        unique_types = torch.unique(keys.flatten())
        assert unique_types.min() >= 0
        max_type = int(unique_types.max())
        sizes = tuple(max_type + 1 for _ in range(order))
        self.n_degs = n_degs
        self.k1_names = ["k1_" + str(ii) for ii in range(1, n_degs + 1)]
        self.k2_names = ["k2_" + str(ii) for ii in range(1, n_degs + 1)]
        k1 = torch.zeros(n_degs, *sizes)
        k2 = torch.zeros(n_degs, *sizes)
        v_0 = torch.zeros(*sizes)
        for key in statistics.keys():
            for ii in range(n_degs):
                k1[ii][key] = statistics[key]["k1s"][self.k1_names[ii]]
                k2[ii][key] = statistics[key]["k2s"][self.k2_names[ii]]
            v_0[key] = statistics[key]["v_0"]
        self.register_buffer("k1s", k1)
        self.register_buffer("k2s", k2)
        self.register_buffer("v_0", v_0)

    def data2parameters(self, data):
        t = self._types(data, self.order)
        k1s = torch.vstack([self.k1s[ii][t] for ii in range(self.n_degs)]).t()
        k2s = torch.vstack([self.k2s[ii][t] for ii in range(self.n_degs)]).t()
        v_0 = self.v_0[t].view(-1, 1)
        return {"k1s": k1s, "k2s": k2s, "v_0": v_0}

    def param_matrix(self, data):
        p = self.data2parameters(data)
        v0 = p["v_0"]
        if v0.ndim > 1:
            v0 = v0[:, 0]
        return torch.cat([v0.reshape(-1, 1), p["k1s"], p["k2s"]], dim=1)

    @staticmethod
    def compute(theta, v_0, k1s, k2s):
        n_k = k1s.shape[1]
        n = torch.arange(1, n_k + 1, dtype=theta.dtype, device=theta.device)
        angles = theta.view(-1, 1) * n.view(1, -1)
        V = k1s * torch.sin(angles) + k2s * torch.cos(angles)
        if v_0.ndim > 1:
            v_0 = v_0[:, 0]
        return V.sum(dim=1) + v_0


class Dihedral(FourierSeries):
    name: Final[str] = "dihedrals"
    _order: Final[int] = 4

    def __init__(self, statistics: Dict, n_degs: int = 3, name: str = "dihedrals") -> None:
        super().__init__(statistics, name=name, n_degs=n_degs, order=self._order)


class Repulsion(_Prior):
    """U = (sigma / r)^6 over a pair list, sigma from a type-pair table
    (prior/repulsion.py:14-140)."""

    name: Final[str] = "repulsion"
    _neighbor_list_name = "fully connected"
    kind = ops.PRIOR_KIND["repulsion"]

    def __init__(self, statistics: Dict) -> None:
        super().__init__()
        keys = torch.tensor(list(statistics.keys()), dtype=torch.long)
        self.allowed_interaction_keys = list(statistics.keys())
        self.order = 2
        unique_types = torch.unique(keys.flatten())
        assert unique_types.min() >= 0
        max_type = int(unique_types.max())
        sigma = torch.zeros(max_type + 1, max_type + 1)
        for key in statistics.keys():
            sigma[key] = statistics[key]["sigma"]
        self.register_buffer("sigma", sigma)

    def data2parameters(self, data):
        return {"sigma": self.sigma[self._types(data, 2)].flatten()}

    def param_matrix(self, data):
        return self.data2parameters(data)["sigma"].reshape(-1, 1)

    @staticmethod
    def compute(x, sigma):
        rr = (sigma / x) * (sigma / x)
        return rr * rr * rr


class _StaticMixin:
    """Pre-gathered per-interaction parameters (the Static* priors of
    mlcg/simulation/specialize_prior.py:49-72): buffers hold one value (row)
    per interaction of the collated simulation batch."""

    def _init_static(self, **params):
        torch.nn.Module.__init__(self)
        self._graph_key = None
        self._graph = None
        self.param_names = []
        for k, v in params.items():
            self.register_buffer(k, v)
            self.param_names.append(k)

    def data2parameters(self, data):
        return {k: getattr(self, k) for k in self.param_names}


class StaticHarmonicBonds(_StaticMixin, HarmonicBonds):
    def __init__(self, **params):
        self._init_static(**params)
        self.order = 2


class StaticHarmonicAngles(_StaticMixin, HarmonicAngles):
    def __init__(self, **params):
        self._init_static(**params)
        self.order = 3


class StaticDihedral(_StaticMixin, Dihedral):
    def __init__(self, n_degs: int = 3, **params):
        self._init_static(**params)
        self.order = 4
        self.n_degs = n_degs

    def param_matrix(self, data):
        p = self.data2parameters(data)
        v0 = p["v_0"]
        if v0.ndim > 1:
            v0 = v0[:, 0]
        return torch.cat([v0.reshape(-1, 1), p["k1s"][:, :self.n_degs],
                          p["k2s"][:, :self.n_degs]], dim=1)


class StaticRepulsion(_StaticMixin, Repulsion):
    def __init__(self, **params):
        self._init_static(**params)
        self.order = 2
