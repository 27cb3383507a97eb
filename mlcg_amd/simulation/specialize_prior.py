"""Specialised (pre-gathered) priors for simulations
(mlcg/simulation/specialize_prior.py:49-206).

``condense_all_priors_for_simulation(priors, data_list)`` replaces every
HarmonicBonds / HarmonicAngles / Dihedral / Repulsion model of a SumOut by one
Static* prior per kind whose buffers hold the per-interaction parameters of
the given configurations, concatenated in configuration order -- the order in
which collation concatenates the neighbour lists -- and merges the neighbour
lists of the condensed priors under the prior's name.  The static form skips
the per-call type-table gather, so the prior kernels read parameters
directly.
"""

from __future__ import annotations

from collections import defaultdict
from copy import deepcopy
from typing import List, Tuple

import torch

from ..nn import (Dihedral, GradientsOut, HarmonicAngles, HarmonicBonds, Repulsion,
                  StaticDihedral, StaticHarmonicAngles, StaticHarmonicBonds, StaticRepulsion,
                  SumOut)

#: prior classes that can be condensed, with their static counterparts
to_reduce = {
    "HarmonicBonds": (HarmonicBonds, StaticHarmonicBonds),
    "HarmonicAngles": (HarmonicAngles, StaticHarmonicAngles),
    "Dihedral": (Dihedral, StaticDihedral),
    "Repulsion": (Repulsion, StaticRepulsion),
}


def condense_prior_for_simulation(target: str, priors: SumOut, data_list: List):
    CLS, STATIC = to_reduce[target]
    condensed_priors = deepcopy(priors)
    condensed_data = deepcopy(data_list)
    names = [k for k, p in priors.models.items()
             if isinstance(p.model, CLS) and not isinstance(p.model, STATIC)]
    if not names:
        return condensed_priors, condensed_data
    n_degs = max([priors.models[k].model.n_degs for k in names]) if CLS is Dihedral else 1
    params = defaultdict(list)
    for ii, data in enumerate(condensed_data):
        mappings = []
        for k in names:
            prior = priors.models[k].model
            pp = prior.data2parameters(data_list[ii])
            for kv, v in pp.items():
                v = v.detach().cpu()
                if v.ndim == 1:
                    v = v.unsqueeze(-1)
                ee = torch.zeros(v.shape[0], n_degs)
                ee[:, :v.shape[1]] = v
                params[kv].append(ee)
            mappings.append(data_list[ii].neighbor_list[k]["index_mapping"])
            data.neighbor_list.pop(k)
        nl = {"tag": f"Static{target}", "order": mappings[0].shape[0],
              "index_mapping": torch.cat(mappings, dim=-1), "cell_shifts": None,
              "rcut": None, "self_interaction": False}
        data.neighbor_list[CLS.name] = nl
    for k in names:
        condensed_priors.models.pop(k)
    out = {}
    for k, v in params.items():
        out[k] = torch.vstack(v) if CLS is Dihedral else torch.cat(v).flatten()
    static = STATIC(n_degs=n_degs, **out) if CLS is Dihedral else STATIC(**out)
    condensed_priors.models[CLS.name] = GradientsOut(static)
    return condensed_priors, condensed_data


def condense_all_priors_for_simulation(priors: SumOut, data_list: List) -> Tuple[SumOut, List]:
    for target in to_reduce:
        priors, data_list = condense_prior_for_simulation(target, priors, data_list)
    return priors, data_list
