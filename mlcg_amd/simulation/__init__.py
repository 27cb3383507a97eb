"""Langevin simulation on the HIP kernels (mlcg/simulation/)."""

from .langevin import LangevinSimulation, sample_maxwell_boltzmann
from .specialize_prior import condense_all_priors_for_simulation

__all__ = ["LangevinSimulation", "sample_maxwell_boltzmann",
           "condense_all_priors_for_simulation"]
