"""Langevin simulation on the HIP kernels (mlcg/simulation/)."""

from .langevin import LangevinSimulation, sample_maxwell_boltzmann
from .parallel_tempering import PTSimulation
from .specialize_prior import condense_all_priors_for_simulation

__all__ = ["LangevinSimulation", "PTSimulation", "sample_maxwell_boltzmann",
           "condense_all_priors_for_simulation"]
