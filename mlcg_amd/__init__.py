"""mlcg_amd -- MI355X-native (gfx950) implementation of mlcg's SchNet CFConv
hot path: radius graph, Gaussian-RBF filter network, CFConv gather/scatter
with hand-derived force backward and force-matching double backward, priors
and the Langevin integrator, behind mlcg's module API."""

from . import library, ops
from ._lib import available, version

# torch.ops.mlcg.radius_cuda / exclusion_pair_to_ptr, as the reference's
# extension registers them; and this library's own model operators, through
# which torch.compile sees the fused energy/force passes
library.register()
library.register_model_ops()

__all__ = ["ops", "available", "version"]
