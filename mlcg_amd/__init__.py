"""mlcg_amd -- MI355X-native (gfx950) implementation of mlcg's SchNet CFConv
hot path: radius graph, Gaussian-RBF filter network, CFConv gather/scatter
with hand-derived force backward and force-matching double backward, priors
and the Langevin integrator, behind mlcg's module API."""

from . import library, ops
from ._lib import available, version

# torch.ops.mlcg.radius_cuda / exclusion_pair_to_ptr, as the reference's
# extension registers them
library.register()

__all__ = ["ops", "available", "version"]
