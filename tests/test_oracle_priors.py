"""Pins the CPU prior oracle (oracle/priors_ref.py) and the BAOAB oracle
(oracle/langevin_ref.py) without a GPU.

  compute_distances / compute_angles_cos   closed forms (3-4-5 triangle,
                                           right, straight and 60-degree angles)
  compute_torsions                         the IUPAC dihedral formula written
                                           independently, and hand-built quarter
                                           turns with the mdtraj sign (the
                                           reference pins it to mdtraj,
                                           tests/unit/geometry/test_internals.py:35-46)
  harmonic / fourier / repulsion energies  closed forms at chosen geometries
  prior forces                             central finite differences (fp64),
                                           zero net force per interaction
  chain_topology                           counts and index ranges
  BAOAB step                               an independent per-component
                                           restatement of langevin.py:100-144
                                           with the same injected noise; free
                                           particle without friction or noise
                                           moves ballistically; vscale and
                                           noisescale closed forms
"""

import math

import numpy as np
import pytest
import torch

from oracle import langevin_ref as L
from oracle import priors_ref as P

D64 = torch.float64


def test_distances_and_angles_closed_forms():
    pos = torch.tensor([[0.0, 0, 0], [3.0, 0, 0], [3.0, 4.0, 0]], dtype=D64)
    d = P.compute_distances(pos, torch.tensor([[0, 1, 0], [1, 2, 2]]))
    assert torch.allclose(d, torch.tensor([3.0, 4.0, 5.0], dtype=D64))
    # angle at bead 1 between 0-1 and 2-1: a right angle
    c = P.compute_angles_cos(pos, torch.tensor([[0], [1], [2]]))
    assert abs(float(c)) < 1e-15
    straight = torch.tensor([[-1.0, 0, 0], [0, 0, 0], [2.0, 0, 0]], dtype=D64)
    assert float(P.compute_angles_cos(straight, torch.tensor([[0], [1], [2]]))) == pytest.approx(-1)
    sixty = torch.tensor([[1.0, 0, 0], [0, 0, 0], [0.5, math.sqrt(3) / 2, 0]], dtype=D64)
    assert float(P.compute_angles_cos(sixty, torch.tensor([[0], [1], [2]]))) == pytest.approx(0.5)


def _iupac(p):
    b1, b2, b3 = p[:, 1] - p[:, 0], p[:, 2] - p[:, 1], p[:, 3] - p[:, 2]
    n1, n2 = np.cross(b1, b2), np.cross(b2, b3)
    return np.arctan2(np.linalg.norm(b2, axis=1) * (b1 * n2).sum(1), (n1 * n2).sum(1))


def test_torsions_match_iupac_formula():
    rng = np.random.default_rng(0)
    p = rng.normal(0, 2.0, (500, 4, 3))
    pos = torch.from_numpy(p.reshape(-1, 3))
    mapping = torch.arange(2000).view(500, 4).t()
    t = P.compute_torsions(pos, mapping).numpy()
    diff = np.angle(np.exp(1j * (t - _iupac(p))))
    assert np.abs(diff).max() < 1e-12


@pytest.mark.parametrize("z,expected", [(1.0, math.pi / 2), (-1.0, -math.pi / 2),
                                        (0.0, 0.0)])
def test_torsion_quarter_turns(z, expected):
    """i at +y, j at origin, k on +x; l rotated about the j-k axis.  With l
    at +y (cis) the torsion is 0; the sign of the quarter turns follows the
    IUPAC / mdtraj convention."""
    l = [1.0, 1.0, 0.0] if z == 0.0 else [1.0, 0.0, z]
    pos = torch.tensor([[0.0, 1.0, 0.0], [0.0, 0, 0], [1.0, 0, 0], l], dtype=D64)
    t = float(P.compute_torsions(pos, torch.tensor([[0], [1], [2], [3]])))
    assert t == pytest.approx(expected, abs=1e-12)
    # independent check of the sign against the formula
    assert t == pytest.approx(float(_iupac(pos.numpy()[None])[0]), abs=1e-12)


def test_energy_closed_forms():
    x = torch.tensor([3.8], dtype=D64)
    assert float(P.harmonic(x, 3.8, 100.0, 0.25)) == 0.25
    assert float(P.harmonic(x + 0.1, 3.8, 100.0)) == pytest.approx(1.0)
    assert float(P.repulsion(torch.tensor([4.0], dtype=D64), 4.0)) == 1.0
    assert float(P.repulsion(torch.tensor([8.0], dtype=D64), 4.0)) == pytest.approx(2 ** -6)
    k1 = torch.tensor([[0.3, -0.2, 0.1]], dtype=D64)
    k2 = torch.tensor([[0.5, 0.7, -0.4]], dtype=D64)
    v0 = torch.tensor([1.5], dtype=D64)
    assert float(P.fourier_series(torch.zeros(1, dtype=D64), v0, k1, k2)) == pytest.approx(
        1.5 + 0.5 + 0.7 - 0.4)
    # theta = pi/2: sin terms 1, 0, -1; cos terms 0, -1, 0
    assert float(P.fourier_series(torch.tensor([math.pi / 2], dtype=D64), v0, k1, k2)) == \
        pytest.approx(1.5 + 0.3 - 0.1 - 0.7)


def _chain(n_frames=3, n=8, seed=1):
    rng = np.random.default_rng(seed)
    steps = rng.normal(size=(n_frames, n, 3))
    steps = 3.8 * steps / np.linalg.norm(steps, axis=-1, keepdims=True)
    return torch.from_numpy(np.cumsum(steps, axis=1).reshape(-1, 3))


def _params(kind, M, seed=2):
    g = torch.Generator().manual_seed(seed)
    if kind in ("bonds", "angles"):
        return {"x0": torch.rand(M, generator=g, dtype=D64) * (3.8 if kind == "bonds" else 1),
                "k": 1 + 10 * torch.rand(M, generator=g, dtype=D64),
                "V0": torch.rand(M, generator=g, dtype=D64)}
    if kind == "dihedrals":
        return {"v_0": torch.rand(M, generator=g, dtype=D64),
                "k1s": torch.randn(M, 3, generator=g, dtype=D64),
                "k2s": torch.randn(M, 3, generator=g, dtype=D64)}
    return {"sigma": 3.0 + torch.rand(M, generator=g, dtype=D64)}


@pytest.mark.parametrize("kind", ["bonds", "angles", "dihedrals", "repulsion"])
def test_prior_forces_finite_differences(kind):
    n_frames, n = 3, 8
    pos = _chain(n_frames, n)
    topo = P.chain_topology(n_frames, n)
    mapping, mb = topo[kind]
    params = _params(kind, mapping.shape[1])
    E, F = P.prior_energy_forces(kind, pos, mapping, mb, n_frames, params)
    h = 1e-6
    Ffd = torch.zeros_like(pos)
    for a in range(pos.shape[0]):
        for c in range(3):
            pp, pm = pos.clone(), pos.clone()
            pp[a, c] += h
            pm[a, c] -= h
            Ffd[a, c] = -(P.prior_energy(kind, pp, mapping, mb, n_frames, params).sum()
                          - P.prior_energy(kind, pm, mapping, mb, n_frames, params).sum()) / (2 * h)
    assert torch.allclose(F, Ffd, rtol=1e-6, atol=1e-7 * float(F.abs().max()))
    for b in range(n_frames):
        assert torch.allclose(F[b * n:(b + 1) * n].sum(0), torch.zeros(3, dtype=D64),
                              atol=1e-9 * float(F.abs().max()))


def test_chain_topology_counts():
    topo = P.chain_topology(2, 10, min_sep=3)
    assert topo["bonds"][0].shape == (2, 18)
    assert topo["angles"][0].shape == (3, 16)
    assert topo["dihedrals"][0].shape == (4, 14)
    m = topo["repulsion"][0]
    assert m.shape[1] == 2 * sum(1 for i in range(10) for j in range(10) if abs(i - j) >= 3)
    assert bool(((m[0] // 10) == (m[1] // 10)).all())
    assert bool(((m[0] - m[1]).abs() >= 3).all())


def test_baoab_matches_per_component_restatement():
    rng = np.random.default_rng(5)
    n = 17
    x = rng.normal(size=(n, 3))
    v = rng.normal(size=(n, 3))
    F = rng.normal(size=(n, 3))
    Fn = rng.normal(size=(n, 3))
    m = rng.uniform(1, 3, n)
    bmr = rng.uniform(0.5, 1.5, n)
    xi = rng.normal(size=(n, 3))
    dt, gamma = 0.004, 1.0
    vs = math.exp(-dt * gamma)
    ns = math.sqrt(1 - vs * vs)
    x1, v1 = L.baoa(torch.from_numpy(x), torch.from_numpy(v), torch.from_numpy(F),
                    torch.from_numpy(m), torch.from_numpy(bmr), dt, vs, ns, torch.from_numpy(xi))
    v2 = L.b(v1, torch.from_numpy(Fn), torch.from_numpy(m), dt)
    for a in range(n):
        for c in range(3):
            vv = v[a, c] + 0.5 * dt * F[a, c] / m[a]
            xx = x[a, c] + vv * dt * 0.5
            vv = vv * vs + ns * bmr[a] * xi[a, c]
            xx = xx + vv * dt * 0.5
            vv = vv + 0.5 * dt * Fn[a, c] / m[a]
            assert float(x1[a, c]) == pytest.approx(xx, rel=1e-14)
            assert float(v2[a, c]) == pytest.approx(vv, rel=1e-14)


def test_baoab_free_particle_ballistic():
    x = torch.zeros(4, 3, dtype=D64)
    v = torch.ones(4, 3, dtype=D64)
    z = torch.zeros(4, 3, dtype=D64)
    m = torch.ones(4, dtype=D64)
    for _ in range(10):
        x, v = L.baoa(x, v, z, m, m, 0.1, 1.0, 0.0, z)
        v = L.b(v, z, m, 0.1)
    assert torch.allclose(x, torch.ones(4, 3, dtype=D64))
    assert torch.allclose(v, torch.ones(4, 3, dtype=D64))


def test_langevin_constants():
    vs, ns = L.constants(dt=0.004, friction=1.0)
    assert vs == pytest.approx(math.exp(-0.004))
    assert vs * vs + ns * ns == pytest.approx(1.0)
    # beta of 300 K in kcal/mol (k_B = 0.0019872041 kcal/mol/K, mol_utils.py:108)
    assert L.beta_of(300.0) == pytest.approx(1.0 / (0.0019872041 * 300.0))
