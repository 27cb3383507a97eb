"""Writes the small golden fixtures under tests/golden/ (run from the repo
root: ``python tests/golden/make_golden.py``).

radius_small.npz  8 frames x 100-bead compact globules (config-3 generator,
                  Rg ~ 12 A), cutoff 15 A, no loops: positions, batch and the
                  canonical edge_index of the C oracle.  Before writing, the
                  edge set is checked against per-frame scipy cKDTree
                  queries (the reference's radius oracle,
                  src/opt_radius/mlcg_opt_radius/utils.py:32-47) away from the
                  cutoff boundary.
schnet_small.pt   3 frames x 9-bead self-avoiding chains, SchNet with 2
                  blocks, hidden 16, 128 filters, 16 RBF on 0-9 A, cosine
                  envelopes, tanh, output MLP 16 -> 8 -> 1: the fp64
                  oracle's energies, forces, force-matching loss and every
                  parameter gradient, plus the state_dict and edge list.  Saved
                  with torch.save of plain tensors (loadable with
                  weights_only=True).
config2_512.pt    the full config-2 training batch (512 frames x 35-bead
                  self-avoiding chains, synthetic.config2()) through the
                  config-2 model (3 blocks, H = F = 128, 50 Gaussian RBF on
                  0-20 A with a cosine envelope, cosine cutoff 20 A, tanh,
                  output MLP 128 -> 64 -> 1; weights random_state_dict(seed
                  20262)): the fp64 oracle's energies, forces, force-matching
                  loss and every parameter gradient (evaluated in 32-frame
                  chunks, R.force_matching_grads_chunked), stored as float32
                  (rounding 6e-8 relative, far inside the 1e-5 / 1e-4
                  tolerances), plus the edge count and a float64 checksum of
                  the positions so that a test can tell the generator still
                  yields the same batch.

``python tests/golden/make_golden.py [name ...]`` writes the named fixtures
(all three by default).
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from mlcg_amd import synthetic  # noqa: E402
from oracle import radius as oracle_radius  # noqa: E402
from oracle import schnet_ref as R  # noqa: E402


def radius_small():
    rng = np.random.default_rng(20263)
    pos3 = synthetic.globule(8, 100, 26.0, rng)
    b = synthetic._flatten(pos3, np.ones((8, 100), np.int64), 20263)
    ei, ovf = oracle_radius.radius_graph(b.pos, 15.0, b.batch, False, 1000)
    assert ovf == 0
    from scipy.spatial import cKDTree

    got = set(map(tuple, ei.T.tolist()))
    for f in range(8):
        idx = np.arange(100 * f, 100 * f + 100)
        p = b.pos[idx].astype(np.float64)
        tree = cKDTree(p)
        for a, hits in enumerate(tree.query_ball_point(p, 15.0 + 1e-4)):
            for h in hits:
                if h == a:
                    continue
                d = np.linalg.norm(p[h] - p[a])
                if abs(d - 15.0) > 1e-4:
                    assert ((idx[a], idx[h]) in got) == (d < 15.0)
    np.savez_compressed(os.path.join(HERE, "radius_small.npz"), pos=b.pos, batch=b.batch,
                        r=np.float64(15.0), edge_index=ei)
    print("radius_small.npz: E =", ei.shape[1])


def schnet_small():
    rng = np.random.default_rng(20262)
    pos3 = synthetic.self_avoiding_walk(3, 9, rng)
    types = rng.integers(1, 21, size=(3, 9))
    b = synthetic._flatten(pos3, types, 20262)
    cfg = dict(num_rbf=16, rbf_lo=0.0, rbf_hi=9.0, rbf_cut="cosine", conv_cut="cosine",
               conv_lo=0.0, conv_hi=9.0, act="tanh", num_blocks=2)
    c = R.SchNetConfig(**cfg)
    sd = R.to_dtype(R.random_state_dict(c, hidden=16, embedding_size=24, out_widths=(8,),
                                        seed=20262, bias_scale=0.2),
                    torch.float64)
    ei, _ = oracle_radius.radius_graph(b.pos, 9.0, b.batch, False, 1000)
    ei = torch.from_numpy(ei)
    pos = torch.from_numpy(b.pos).double()
    tt = torch.from_numpy(b.atom_types)
    bb = torch.from_numpy(b.batch)
    fref = torch.from_numpy(rng.standard_normal((27, 3)))
    E, F = R.schnet_energy_forces(sd, c, pos, tt, bb, ei, 3)
    loss, _, _, grads = R.force_matching_grads(sd, c, pos, tt, bb, ei, 3, fref)
    torch.save({"cfg": cfg, "state_dict": sd, "pos": pos, "types": tt, "batch": bb,
                "edge_index": ei, "n_frames": torch.tensor(3), "energy": E.detach(),
                "forces": F.detach(), "forces_ref": fref, "loss": loss,
                "grads": {k: v.detach() for k, v in grads.items()}},
               os.path.join(HERE, "schnet_small.pt"))
    print("schnet_small.pt: E =", ei.shape[1], "loss", float(loss))


CONFIG2_SEED = 20262


def config2_512():
    import time

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    b = synthetic.config2()
    cfg = R.SchNetConfig(num_rbf=50, rbf_lo=0.0, rbf_hi=20.0, rbf_cut="cosine",
                         conv_cut="cosine", conv_lo=0.0, conv_hi=20.0, act="tanh", num_blocks=3)
    sd = R.random_state_dict(cfg, seed=CONFIG2_SEED)
    ei, ovf = oracle_radius.radius_graph(b.pos, 20.0, b.batch, False, 1000)
    assert ovf == 0
    t0 = time.time()
    loss, E, F, grads = R.force_matching_grads_chunked(
        R.to_dtype(sd, torch.float64), cfg, torch.from_numpy(b.pos).double(),
        torch.from_numpy(b.atom_types), torch.from_numpy(b.batch), torch.from_numpy(ei),
        b.n_frames, torch.from_numpy(b.forces).double(), frames_per_chunk=32)
    torch.save({"seed": torch.tensor(CONFIG2_SEED), "n_frames": torch.tensor(b.n_frames),
                "num_edges": torch.tensor(ei.shape[1]),
                "pos_checksum": torch.tensor(float(np.abs(b.pos.astype(np.float64)).sum()),
                                             dtype=torch.float64),
                "loss": loss.double(), "energy": E.float(), "forces": F.float(),
                "grads": {k: v.float() for k, v in grads.items()}},
               os.path.join(HERE, "config2_512.pt"))
    print("config2_512.pt: E =", ei.shape[1], "loss", float(loss),
          f"({time.time() - t0:.0f} s)")


if __name__ == "__main__":
    names = sys.argv[1:] or ["radius_small", "schnet_small", "config2_512"]
    for name in names:
        globals()[name]()
