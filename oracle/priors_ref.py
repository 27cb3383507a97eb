"""CPU restatement of mlcg's prior energies -- TEST INFRASTRUCTURE.

Energies follow the reference op by op (any dtype); forces come from
torch.autograd, as GradientsOut does (mlcg/nn/gradients.py:208-226).  Per-frame
sums replace torch_geometric.utils.scatter(..., reduce="sum") with index_add_.

  compute_distances   internal_coordinates.py:73-100
  compute_angles_cos  internal_coordinates.py:146-183
  compute_torsions    internal_coordinates.py:187-252
  harmonic            Harmonic.compute, prior/harmonic.py:119-120 (no 1/2)
  fourier_series      FourierSeries.compute, prior/fourier_series.py:160-198
  repulsion           Repulsion.compute, prior/repulsion.py:136-140

Parity pins (tests/test_oracle_priors.py):
  distances / cos    closed forms on hand-built geometries (3-4-5 triangle,
                     right and straight angles)
  torsions           the IUPAC/mdtraj dihedral formula
                     atan2(|b2| b1.(b2 x b3), (b1 x b2).(b2 x b3)) written
                     independently, plus the signed quarter turns of a
                     hand-built geometry (the reference checks against mdtraj,
                     tests/unit/geometry/test_internals.py:35-46)
  energies           closed forms at chosen geometries (x = x0 gives V0,
                     sigma = r gives 1, theta = 0 gives sum k2 + v0)
  forces             central finite differences in fp64; zero net force per
                     interaction
"""

from __future__ import annotations

from typing import Optional

import torch


def compute_distances(pos: torch.Tensor, mapping: torch.Tensor) -> torch.Tensor:
    dr = pos[mapping[1]] - pos[mapping[0]]
    return dr.norm(p=2, dim=1)


def compute_angles_cos(pos: torch.Tensor, mapping: torch.Tensor) -> torch.Tensor:
    dr1 = pos[mapping[0]] - pos[mapping[1]]
    dr2 = pos[mapping[2]] - pos[mapping[1]]
    return (dr1 * dr2).sum(dim=1) / dr1.norm(p=2, dim=1) / dr2.norm(p=2, dim=1)


def compute_torsions(pos: torch.Tensor, mapping: torch.Tensor) -> torch.Tensor:
    dr1 = pos[mapping[1]] - pos[mapping[0]]
    dr2 = pos[mapping[2]] - pos[mapping[1]]
    dr3 = pos[mapping[3]] - pos[mapping[2]]
    dr1 = dr1 / dr1.norm(p=2, dim=1)[:, None]
    dr2 = dr2 / dr2.norm(p=2, dim=1)[:, None]
    dr3 = dr3 / dr3.norm(p=2, dim=1)[:, None]
    n1 = torch.cross(dr1, dr2, dim=1)
    n2 = torch.cross(dr2, dr3, dim=1)
    m1 = torch.cross(n1, dr2, dim=1)
    y = torch.sum(m1 * n2, dim=-1)
    x = torch.sum(n1 * n2, dim=-1)
    return torch.atan2(-y, x)


def harmonic(x, x0, k, V0=0.0):
    return k * (x - x0) ** 2 + V0


def fourier_series(theta, v_0, k1s, k2s):
    n_k = k1s.shape[1]
    n_degs = torch.arange(1, n_k + 1, dtype=theta.dtype)
    angles = theta.view(-1, 1) * n_degs.view(1, -1)
    V = k1s * torch.sin(angles) + k2s * torch.cos(angles)
    if v_0.ndim > 1:
        v_0 = v_0[:, 0]
    return V.sum(dim=1) + v_0


def repulsion(x, sigma):
    rr = (sigma / x) * (sigma / x)
    return rr * rr * rr


def prior_energy(kind: str, pos: torch.Tensor, mapping: torch.Tensor,
                 mapping_batch: torch.Tensor, n_frames: int, params: dict) -> torch.Tensor:
    """Per-frame energies [B] of one prior.

    kind: "bonds" / "angles" (params x0, k, V0 per interaction),
          "dihedrals" (v_0 [M], k1s [M, n], k2s [M, n]), "repulsion" (sigma [M]).
    """
    if kind == "bonds":
        y = harmonic(compute_distances(pos, mapping), params["x0"], params["k"],
                     params.get("V0", 0.0))
    elif kind == "angles":
        y = harmonic(compute_angles_cos(pos, mapping), params["x0"], params["k"],
                     params.get("V0", 0.0))
    elif kind == "dihedrals":
        y = fourier_series(compute_torsions(pos, mapping), params["v_0"], params["k1s"],
                           params["k2s"])
    elif kind == "repulsion":
        y = repulsion(compute_distances(pos, mapping), params["sigma"])
    else:
        raise ValueError(kind)
    return torch.zeros(n_frames, dtype=y.dtype).index_add_(0, mapping_batch, y)


def prior_energy_forces(kind, pos, mapping, mapping_batch, n_frames, params):
    pos = pos.detach().requires_grad_(True)
    E = prior_energy(kind, pos, mapping, mapping_batch, n_frames, params)
    (g,) = torch.autograd.grad(E.sum(), pos)
    return E.detach(), -g


def chain_topology(n_frames: int, n_beads: int, min_sep: Optional[int] = 3):
    """Bonds (i, i+1), angles (i, i+1, i+2), dihedrals (i..i+3) and the
    repulsion pair list of every frame of a linear chain, as [order, M]
    int64 index maps with mapping_batch.  Repulsion uses all ordered pairs
    with |i - j| >= min_sep, the builder's choice for config 5 (the
    reference's "fully connected" list, topology.py:131-135, minus the bonded
    neighbours)."""
    def stack(order):
        base = torch.arange(n_beads - order + 1)
        idx = torch.stack([base + s for s in range(order)])
        maps = [idx + f * n_beads for f in range(n_frames)]
        mb = torch.arange(n_frames).repeat_interleave(idx.shape[1])
        return torch.cat(maps, dim=1), mb

    out = {"bonds": stack(2), "angles": stack(3), "dihedrals": stack(4)}
    ii, jj = torch.meshgrid(torch.arange(n_beads), torch.arange(n_beads), indexing="ij")
    keep = (ii - jj).abs() >= (min_sep or 1)
    pij = torch.stack([ii[keep], jj[keep]])
    maps = [pij + f * n_beads for f in range(n_frames)]
    out["repulsion"] = (torch.cat(maps, dim=1),
                        torch.arange(n_frames).repeat_interleave(pij.shape[1]))
    return out
