"""CPU oracle for the mlcg SchNet/CFConv hot path -- TEST INFRASTRUCTURE.

This package restates the reference algorithms (ClementiGroup/mlcg, cited by
file:line in each function) on the CPU so that the HIP kernels of
``mlcg_amd`` can be checked against them.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker or the timed CPU baseline; the product
(``mlcg_amd``) never imports, links or calls anything here.

Contents
  radius       -- brute-force per-frame radius graph (C, exact fp32 predicate)
  schnet_ref   -- SchNet / CFConv / Gaussian RBF / cosine cutoff / MLP,
                  GradientsOut forces and the force-matching double backward
                  through torch.autograd (PyG replaced by index_select /
                  index_add_)
  priors_ref   -- harmonic bonds and angles, Fourier dihedrals, repulsion
  langevin_ref -- BAOAB Langevin step

Parity status of every function (what pins it) is listed in each module's
docstring.  Functions pinned only by the restatement itself are marked
"parity unpinned".
"""
