"""Parallel tempering (replica exchange) on the BAOAB driver
(mlcg/simulation/parallel_tempering.py:24-566).

``PTSimulation(exchange_interval=..., **LangevinSimulation arguments)`` runs
every configuration at every temperature of ``betas`` (largest beta first):
simulation slot r * n_indep + i holds configuration i at betas[r].  Every
``exchange_interval`` steps it proposes exchanges between directly adjacent
temperatures, alternating the pairs (0,1), (2,3), ... and (1,2), (3,4), ...,
accepts a pair with the Metropolis probability
min(1, exp((U_a - U_b)(beta_a - beta_b))), and swaps the two slots'
configurations, rescaling the velocities by sqrt(beta_new / beta_old) as
the reference's code does (parallel_tempering.py:360-520, the factor at
484-497), so that a run reproduces a reference run.  The reference's
docstring (433-435) states the inverse, sqrt(beta_old / beta_new), which
keeps a moved configuration's kinetic temperature consistent with its new
slot (equipartition); ``reference_velocity_scaling=False`` applies that
factor instead.  The forces travel with the configurations
(a force depends on the configuration only), so the next half-kick uses the
force of the configuration it moves.  `acceptance_matrix[a, b]` counts the
accepted (a < b) and rejected (a > b) exchanges between temperatures a and b.
The exchange runs on the host between steps, so it also works with
``capture=True`` (the captured step is replayed around it).
"""

from __future__ import annotations

from typing import List, Tuple

import numpy as np
import torch

from .langevin import LangevinSimulation


class PTSimulation(LangevinSimulation):
    def __init__(self, exchange_interval: int = 100,
                 reference_velocity_scaling: bool = True, **kwargs):
        super().__init__(**kwargs)
        if exchange_interval < 1:
            raise ValueError("exchange_interval must be positive")
        self.exchange_interval = int(exchange_interval)
        # True (the default): a configuration moving from beta_old to beta_new
        # has its velocities scaled by sqrt(beta_new / beta_old), as the
        # reference's code does (484-497); False: by sqrt(beta_old / beta_new),
        # the factor the reference's docstring states (433-435)
        self.reference_velocity_scaling = bool(reference_velocity_scaling)
        self._hook = self.detect_and_exchange_replicas
        self._hook_interval = self.exchange_interval
        self._rng = torch.Generator().manual_seed(self.random_seed + 1)

    def attach_model_and_configurations(self, model: torch.nn.Module, configurations: List,
                                        betas: List[float]):
        if not isinstance(betas, (list, tuple)) or len(betas) < 2:
            raise ValueError(f"Parallel tempering requires multiple temperatures, but only "
                             f"{betas} was supplied.")
        if not all(b > 0 and np.isfinite(b) for b in betas):
            raise ValueError(f"All betas must be positive, but {betas} contains an illegal value.")
        if list(betas) != sorted(betas, reverse=True):
            raise ValueError("Betas must be in order of increasing temperature.")
        self.n_indep_sims = len(configurations)
        self.n_replicas = len(betas)
        extended = [c.clone() for _ in betas for c in configurations]
        ext_betas = [float(b) for b in betas for _ in configurations]
        super().attach_model_and_configurations(model, extended, ext_betas)
        n = self.n_indep_sims

        def pairs(first):
            a = [torch.arange(n) + r * n for r in range(first, self.n_replicas - 1, 2)]
            return torch.cat(a), torch.cat(a) + n

        self._even_pairs = pairs(0)
        self._odd_pairs = pairs(1) if self.n_replicas > 2 else self._even_pairs
        self._propose_even_pairs = True
        self.pair_to_beta_idx = torch.arange(self.n_replicas).repeat_interleave(n)
        self.acceptance_matrix = torch.zeros(self.n_replicas, self.n_replicas)
        self.exchange_attempts = 0
        self.exchange_approved = 0

    def _detect_exchange(self, potential: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Approved (a, b) slot pairs of this round, and the statistics update
        (parallel_tempering.py:377-440)."""
        pair_a, pair_b = self._even_pairs if self._propose_even_pairs else self._odd_pairs
        u = potential.detach().double().cpu()
        beta = self.beta.double().cpu()
        p_pair = (u[pair_a] - u[pair_b]) * (beta[pair_a] - beta[pair_b])
        approved = torch.log(torch.rand(len(p_pair), generator=self._rng,
                                        dtype=torch.float64)) < p_pair
        self.exchange_attempts += len(pair_a)
        self.exchange_approved += int(approved.sum())
        ba, bb = self.pair_to_beta_idx[pair_a], self.pair_to_beta_idx[pair_b]
        for a_, b_, ok in zip(ba.tolist(), bb.tolist(), approved.tolist()):
            if ok:
                self.acceptance_matrix[a_, b_] += 1
            else:
                self.acceptance_matrix[b_, a_] += 1
        return pair_a[approved], pair_b[approved]

    def _perform_exchange(self, x, v, F, potential, pair_a, pair_b) -> None:
        """Swaps the configurations of the approved slot pairs in place,
        velocities rescaled by the reference code's sqrt(beta_new / beta_old)
        (parallel_tempering.py:442-520), or by sqrt(beta_old / beta_new) with
        reference_velocity_scaling=False."""
        if len(pair_a) == 0:
            return
        dev = x.device
        a = pair_a.to(dev)
        b = pair_b.to(dev)
        s = self.n_sims
        x3, v3, f3 = (t.view(s, self.n_atoms, 3) for t in (x, v, F))
        beta = self.beta.to(dev)
        # b's configuration moves into slot a: v sqrt(beta_a / beta_b) (the
        # reference code's factor), or v sqrt(beta_b / beta_a) when asked for
        ratio = beta[a] / beta[b] if self.reference_velocity_scaling else beta[b] / beta[a]
        scale_ba = torch.sqrt(ratio).view(-1, 1, 1).to(v.dtype)
        xa, va, fa, ua = x3[a].clone(), v3[a].clone(), f3[a].clone(), potential[a].clone()
        x3[a] = x3[b]
        x3[b] = xa
        v3[a] = v3[b] * scale_ba
        v3[b] = va / scale_ba
        f3[a] = f3[b]
        f3[b] = fa
        potential[a] = potential[b]
        potential[b] = ua

    def detect_and_exchange_replicas(self, x, v, F, potential) -> None:
        pair_a, pair_b = self._detect_exchange(potential)
        self._perform_exchange(x, v, F, potential, pair_a, pair_b)
        self._propose_even_pairs = not self._propose_even_pairs

    def get_replica_info(self, replica_num: int = 0) -> dict:
        """The beta and the slot indices of one temperature (parallel_tempering.py:329-358)."""
        if not 0 <= replica_num < self.n_replicas:
            raise ValueError(f"replica_num must be in [0, {self.n_replicas})")
        n = self.n_indep_sims
        return {"beta": float(self.beta[replica_num * n]),
                "indices": list(range(replica_num * n, (replica_num + 1) * n))}
