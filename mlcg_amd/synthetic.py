"""Seeded synthetic coarse-grained inputs for the benchmark configurations.

Each generator is vectorised over frames with numpy and returns float32
positions; seeds follow ``20260 + config_index``.

  config 1: random walk, 3.8 A steps along normalised N(0, I) directions plus
            N(0, 0.3 A) jitter; types = bead index 1..n
  config 2/5: self-avoiding walk, 3.8 A bonds, bond angle ~ N(100 deg, 15 deg)
            clipped to (0, 180), dihedral ~ U(-pi, pi); a bead closer than
            4.0 A to an earlier non-adjacent bead is re-drawn; types U{1..20}
  config 3/4: compact globule, 3.8 A random-walk steps confined (by
            rejection) to a sphere of radius R (config 3: R = 26 A, giving
            Rg ~ 12 A; config 4: R = 34 A with a 4.0 A excluded volume, giving
            ~50 neighbours per bead at 15 A)
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

BOND = 3.8
SAW_EXCLUSION = 4.0


def seed_for(config_index: int) -> int:
    return 20260 + config_index


def _unit(v):
    return v / np.linalg.norm(v, axis=-1, keepdims=True)


def random_walk(n_frames: int, n_beads: int, rng: np.random.Generator,
                jitter: float = 0.3) -> np.ndarray:
    steps = _unit(rng.standard_normal((n_frames, n_beads - 1, 3))) * BOND
    pos = np.zeros((n_frames, n_beads, 3))
    pos[:, 1:] = np.cumsum(steps, axis=1)
    pos += rng.normal(0.0, jitter, size=pos.shape)
    return pos.astype(np.float32)


def _place(a, b, c, bond, angle, dihedral):
    """NeRF: position d with |cd| = bond, angle(b, c, d) = angle and
    dihedral(a, b, c, d) = dihedral (arrays over frames)."""
    bc = _unit(c - b)
    n = np.cross(b - a, bc)
    n = _unit(n)
    m = np.cross(n, bc)
    d2 = np.stack([-bond * np.cos(angle),
                   bond * np.sin(angle) * np.cos(dihedral),
                   bond * np.sin(angle) * np.sin(dihedral)], axis=-1)
    return c + d2[..., 0:1] * bc + d2[..., 1:2] * m + d2[..., 2:3] * n


def self_avoiding_walk(n_frames: int, n_beads: int, rng: np.random.Generator,
                       max_tries: int = 200) -> np.ndarray:
    pos = np.zeros((n_frames, n_beads, 3))
    pos[:, 1] = [BOND, 0.0, 0.0]
    ang = np.deg2rad(np.clip(rng.normal(100.0, 15.0, n_frames), 1.0, 179.0))
    pos[:, 2] = pos[:, 1] + BOND * np.stack(
        [-np.cos(ang), np.sin(ang), np.zeros(n_frames)], axis=-1)
    # a virtual bead before 0 makes the first dihedral well defined
    virtual = np.tile(np.array([0.0, 1.0, 0.0]), (n_frames, 1))
    for k in range(3, n_beads):
        todo = np.arange(n_frames)
        new = np.zeros((n_frames, 3))
        for _ in range(max_tries):
            m = todo.size
            angle = np.deg2rad(np.clip(rng.normal(100.0, 15.0, m), 1.0, 179.0))
            dih = rng.uniform(-np.pi, np.pi, m)
            a = pos[todo, k - 3] if k >= 3 else virtual[todo]
            cand = _place(a, pos[todo, k - 2], pos[todo, k - 1], BOND, angle, dih)
            if k >= 3:
                dd = np.linalg.norm(pos[todo, : k - 2] - cand[:, None, :], axis=-1)
                ok = (dd >= SAW_EXCLUSION).all(axis=1)
            else:
                ok = np.ones(m, bool)
            new[todo[ok]] = cand[ok]
            todo = todo[~ok]
            if todo.size == 0:
                break
        if todo.size:  # accept the last candidates (rare dead ends)
            new[todo] = cand[~ok]
        pos[:, k] = new
    pos -= pos.mean(axis=1, keepdims=True)
    return pos.astype(np.float32)


def globule(n_frames: int, n_beads: int, radius: float, rng: np.random.Generator,
            max_tries: int = 64, exclusion: float = 0.0, candidates: int = 16) -> np.ndarray:
    """Random walk of 3.8 A steps confined to a sphere of `radius` (and, with
    `exclusion` > 0, keeping every bead at least that far from all earlier
    non-adjacent beads).  The first round draws one trial step per frame,
    later rounds `candidates` per unfinished frame, keeping the first
    acceptable one; a frame that finds none after `max_tries` rounds keeps a
    trial that satisfies the sphere only (rare dead ends)."""
    pos = np.zeros((n_frames, n_beads, 3))
    pos[:, 0] = _unit(rng.standard_normal((n_frames, 3))) * radius * 0.5 * rng.uniform(
        0, 1, (n_frames, 1))
    for k in range(1, n_beads):
        todo = np.arange(n_frames)
        new = np.zeros((n_frames, 3))
        last = None
        for attempt in range(max_tries):
            m = todo.size
            c = 1 if attempt == 0 else candidates
            cand = pos[todo, k - 1][:, None, :] + _unit(
                rng.standard_normal((m, c, 3))) * BOND
            ok = np.linalg.norm(cand, axis=-1) <= radius
            last = (todo, cand, ok)
            if exclusion > 0 and k >= 2:
                # squared distances to all earlier non-adjacent beads through
                # one batched product: |p|^2 + |c|^2 - 2 p.c
                prev = pos[todo, : k - 1]
                d2 = ((prev * prev).sum(-1)[:, None, :] + (cand * cand).sum(-1)[:, :, None]
                      - 2.0 * np.matmul(cand, prev.transpose(0, 2, 1)))
                ok &= (d2 >= exclusion * exclusion).all(axis=2)
            anyok = ok.any(axis=1)
            first = ok.argmax(axis=1)
            sel = np.nonzero(anyok)[0]
            new[todo[sel]] = cand[sel, first[sel]]
            todo = todo[~anyok]
            if todo.size == 0:
                break
        if todo.size:  # dead end: keep the bond length and the sphere
            t0, cand, ok_sphere = last
            idx = np.searchsorted(t0, todo)
            pick = np.where(ok_sphere[idx].any(axis=1), ok_sphere[idx].argmax(axis=1), 0)
            new[todo] = cand[idx, pick]
        pos[:, k] = new
    return pos.astype(np.float32)


@dataclass
class Batch:
    """A batch of frames flattened the way AtomicData collation does."""

    pos: np.ndarray        # [N, 3] float32
    atom_types: np.ndarray  # [N] int64
    batch: np.ndarray      # [N] int64
    n_atoms: np.ndarray    # [B] int64
    forces: Optional[np.ndarray] = None  # [N, 3] reference forces
    seed: int = 0

    @property
    def n_frames(self) -> int:
        return int(self.n_atoms.shape[0])

    def to_torch(self, device="cpu"):
        import torch

        from .data import AtomicData

        kw = dict(pos=torch.from_numpy(self.pos).to(device),
                  atom_types=torch.from_numpy(self.atom_types).to(device),
                  batch=torch.from_numpy(self.batch).to(device),
                  n_atoms=torch.from_numpy(self.n_atoms).to(device))
        if self.forces is not None:
            kw["forces"] = torch.from_numpy(self.forces).to(device)
        return AtomicData(**kw)


def _flatten(pos3: np.ndarray, types: np.ndarray, seed: int,
             forces: Optional[np.ndarray] = None) -> Batch:
    B, n, _ = pos3.shape
    return Batch(pos=np.ascontiguousarray(pos3.reshape(B * n, 3), dtype=np.float32),
                 atom_types=types.reshape(-1).astype(np.int64),
                 batch=np.repeat(np.arange(B, dtype=np.int64), n),
                 n_atoms=np.full(B, n, dtype=np.int64), forces=forces, seed=seed)


def config1(n_frames: int = 32, n_beads: int = 10) -> Batch:
    seed = seed_for(1)
    rng = np.random.default_rng(seed)
    pos = random_walk(n_frames, n_beads, rng)
    types = np.tile(np.arange(1, n_beads + 1), (n_frames, 1))
    return _flatten(pos, types, seed)


def config2(n_frames: int = 512, n_beads: int = 35) -> Batch:
    seed = seed_for(2)
    rng = np.random.default_rng(seed)
    pos = self_avoiding_walk(n_frames, n_beads, rng)
    types = rng.integers(1, 21, size=(n_frames, n_beads))
    forces = rng.standard_normal((n_frames * n_beads, 3)).astype(np.float32)
    return _flatten(pos, types, seed, forces)


def config3(n_frames: int = 2048, n_beads: int = 100, radius: float = 26.0) -> Batch:
    seed = seed_for(3)
    rng = np.random.default_rng(seed)
    pos = globule(n_frames, n_beads, radius, rng)
    types = rng.integers(1, 21, size=(n_frames, n_beads))
    return _flatten(pos, types, seed)


def config4(n_frames: int = 256, n_beads: int = 500, radius: float = 34.0) -> Batch:
    seed = seed_for(4)
    rng = np.random.default_rng(seed)
    pos = globule(n_frames, n_beads, radius, rng, exclusion=SAW_EXCLUSION)
    types = rng.integers(1, 21, size=(n_frames, n_beads))
    forces = rng.standard_normal((n_frames * n_beads, 3)).astype(np.float32)
    return _flatten(pos, types, seed, forces)


def config5(n_frames: int = 100, n_beads: int = 268) -> Batch:
    seed = seed_for(5)
    rng = np.random.default_rng(seed)
    pos = self_avoiding_walk(n_frames, n_beads, rng)
    types = rng.integers(1, 21, size=(n_frames, n_beads))
    return _flatten(pos, types, seed)


def radius_of_gyration(pos3: np.ndarray) -> np.ndarray:
    c = pos3 - pos3.mean(axis=1, keepdims=True)
    return np.sqrt((c ** 2).sum(-1).mean(-1))


# ---------------------------------------------------------------------------
# Config 5: priors and topology of the CG Langevin workload

#: builder-chosen prior constants for config 5 (the configuration fixes only
#: the bond and repulsion constants; the angle, dihedral and pair-set choices
#: are recorded here)
CONFIG5_PRIORS = {
    "bonds": {"k": 100.0, "x_0": 3.8},
    "angles": {"k": 10.0, "theta_0_deg": 100.0},
    "dihedrals": {"k1s": (0.2, 0.1, 0.05), "k2s": (0.3, -0.1, 0.05), "v_0": 0.0},
    "repulsion": {"sigma": 4.0, "min_separation": 3},
    "masses_amu": 12.0,
    "temperature_K": 300.0,
    "dt_ps": 0.004,
    "friction_per_ps": 1.0,
}


def chain_neighbor_lists(n_beads: int, min_separation: int = 3):
    """Index maps of one linear chain: bonds (i, i+1), angles (i..i+2),
    dihedrals (i..i+3) and the repulsion pairs |i - j| >= min_separation
    (ordered, both directions, as the reference's fully connected list)."""
    import torch

    def stack(order):
        base = torch.arange(n_beads - order + 1)
        return torch.stack([base + s for s in range(order)])

    ii, jj = torch.meshgrid(torch.arange(n_beads), torch.arange(n_beads), indexing="ij")
    keep = (ii - jj).abs() >= min_separation
    nl = {"bonds": stack(2), "angles": stack(3), "dihedrals": stack(4),
          "repulsion": torch.stack([ii[keep], jj[keep]])}
    return {k: {"index_mapping": v, "order": v.shape[0]} for k, v in nl.items()}


def config5_prior_models(n_types: int = 21):
    """HarmonicBonds, HarmonicAngles, Dihedral (3 terms) and Repulsion with the
    CONFIG5_PRIORS constants for every type combination (types < n_types).
    The modules are built from one statistics key and their type tables then
    filled whole, which avoids a Python loop over n_types**4 dihedral keys."""
    import math

    from . import nn

    c = CONFIG5_PRIORS
    top = n_types - 1
    cos0 = math.cos(math.radians(c["angles"]["theta_0_deg"]))
    d = c["dihedrals"]
    mods = {
        "bonds": nn.HarmonicBonds({(top, top): {"x_0": c["bonds"]["x_0"],
                                                "k": c["bonds"]["k"]}}),
        "angles": nn.HarmonicAngles({(top,) * 3: {"x_0": cos0, "k": c["angles"]["k"]}}),
        "dihedrals": nn.Dihedral(
            {(top,) * 4: {"k1s": {f"k1_{i + 1}": v for i, v in enumerate(d["k1s"])},
                          "k2s": {f"k2_{i + 1}": v for i, v in enumerate(d["k2s"])},
                          "v_0": d["v_0"]}}, n_degs=3),
        "repulsion": nn.Repulsion({(top, top): {"sigma": c["repulsion"]["sigma"]}}),
    }
    fill_config5_prior_constants(mods)
    return mods


def fill_config5_prior_constants(mods) -> None:
    """Fills the type tables of the config-5 prior modules (as made by
    config5_prior_models) with the CONFIG5_PRIORS constants, in the tables'
    own dtype: after a move to float64 this makes them the exact decimal
    constants rather than their float32 roundings."""
    import math

    c = CONFIG5_PRIORS
    mods["bonds"].x_0.fill_(c["bonds"]["x_0"])
    mods["bonds"].k.fill_(c["bonds"]["k"])
    mods["angles"].x_0.fill_(math.cos(math.radians(c["angles"]["theta_0_deg"])))
    mods["angles"].k.fill_(c["angles"]["k"])
    d = c["dihedrals"]
    for i in range(3):
        mods["dihedrals"].k1s[i].fill_(d["k1s"][i])
        mods["dihedrals"].k2s[i].fill_(d["k2s"][i])
    mods["dihedrals"].v_0.fill_(d["v_0"])
    mods["repulsion"].sigma.fill_(c["repulsion"]["sigma"])


def config5_configurations(n_frames: int = 100, n_beads: int = 268):
    """AtomicData frames of config 5 with masses and the chain neighbour lists."""
    import torch

    from .data import AtomicData

    b = config5(n_frames, n_beads)
    nls = chain_neighbor_lists(n_beads, CONFIG5_PRIORS["repulsion"]["min_separation"])
    m = CONFIG5_PRIORS["masses_amu"] / 418.4
    out = []
    for f in range(n_frames):
        sl = slice(f * n_beads, (f + 1) * n_beads)
        out.append(AtomicData(pos=torch.from_numpy(b.pos[sl].copy()),
                              atom_types=torch.from_numpy(b.atom_types[sl].copy()),
                              masses=torch.full((n_beads,), m),
                              n_atoms=torch.tensor([n_beads]),
                              neighbor_list={k: dict(v) for k, v in nls.items()}))
    return out
