"""CPU restatement of the BAOAB Langevin step -- TEST INFRASTRUCTURE.

Follows LangevinSimulation.timestep (mlcg/simulation/langevin.py:100-144) op
by op, with the O-step noise passed in (the reference draws it with
torch.randn, langevin.py:129-134), and the constants of langevin.py:75-76 and
176-180.  Pinned in tests/test_oracle_priors.py by a per-component scalar
restatement, the ballistic free particle and the closed-form constants.
"""

from __future__ import annotations

import math

import torch

KB_KCAL = 0.0019872041  # kcal/mol/K (mlcg/mol_utils.py:108)


def constants(dt: float, friction: float):
    vscale = math.exp(-dt * friction)
    return vscale, math.sqrt(1 - vscale * vscale)


def beta_of(temperature: float) -> float:
    return 1.0 / (KB_KCAL * temperature)


def baoa(x, v, forces, masses, beta_mass_ratio, dt, vscale, noisescale, noise):
    """B, A, O, A of langevin.py:123-137; returns new (x, v)."""
    v_new = v + 0.5 * dt * forces / masses[:, None]
    x_new = x + v_new * dt * 0.5
    v_new = v_new * vscale + noisescale * (beta_mass_ratio[:, None] * noise)
    x_new = x_new + v_new * dt * 0.5
    return x_new, v_new


def b(v, forces, masses, dt):
    """Final B of langevin.py:141."""
    return v + 0.5 * dt * forces / masses[:, None]
