"""CPU restatement of mlcg's SchNet energy/force path -- TEST INFRASTRUCTURE.

Each function follows the reference op by op (fp32 or fp64, whatever dtype
the inputs have); PyG's MessagePassing/scatter are replaced by
``index_select`` + ``index_add_`` with the same edge order, and autograd
supplies forces (GradientsOut) and the force-matching double backward.

Parameters come from a ``state_dict`` in the reference's key layout
(``interaction_blocks.{b}.conv.filter_network.layers.0.weight`` ...), so the
oracle and the HIP model can be loaded from the same dict.

Parity pins (besides the restatement itself):
  cosine_cutoff   -- endpoint values of tests/unit/nn/test_cutoff.py:27-42
  gaussian_rbf    -- e_k(mu_k) == C(mu_k); offsets/coeff closed forms
  expnormal_rbf   -- equals gaussian_rbf of u = exp(alpha (lo - d)) with
                     offsets = means, coeff = -beta; e_k == C where u == mu_k;
                     means/betas closed forms (exp_normal.py:80-94)
  basis gradients -- central finite differences in fp64 of the energy and of
                     the force loss with respect to the basis parameters
  schnet_energy   -- two-bead closed form; translation/rotation/permutation
                     invariance; sum_i F_i == 0 per frame
  aggregate       -- per-receiver Python loops over the edge list ("add",
                     "mean", a receiver without messages) on a small graph
  forces          -- central finite differences in fp64
  force_matching  -- torch.autograd.gradgradcheck-style finite differences
                     of the force loss with respect to parameters (fp64)
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch


# --------------------------------------------------------------------------
# Elementary pieces

def identity_cutoff(d: torch.Tensor) -> torch.Tensor:
    """IdentityCutoff.forward (mlcg/nn/cutoff.py:59-72)."""
    return torch.ones_like(d)


def cosine_cutoff(d: torch.Tensor, lo: float, hi: float) -> torch.Tensor:
    """CosineCutoff.forward (mlcg/nn/cutoff.py:110-153)."""
    if lo > 0:
        c = 0.5 * (torch.cos(math.pi * (2 * (d - lo) / (hi - lo) + 1.0)) + 1.0)
        c = c * (d < hi).to(d.dtype)
        c = c * (d > lo).to(d.dtype)
        return c
    c = 0.5 * (torch.cos(d * math.pi / hi) + 1.0)
    return c * (d < hi).to(d.dtype)


@dataclass
class Cutoff:
    kind: str  # "identity" | "cosine"
    lo: float
    hi: float

    def __call__(self, d: torch.Tensor) -> torch.Tensor:
        if self.kind == "identity":
            return identity_cutoff(d)
        return cosine_cutoff(d, self.lo, self.hi)


def gaussian_params(lo: float, hi: float, num_rbf: int, dtype=torch.float32):
    """GaussianBasis._initial_params (mlcg/nn/radial_basis/gaussian.py:64-75)."""
    offset = torch.linspace(lo, hi, num_rbf)
    coeff = -0.5 / (offset[1] - offset[0]) ** 2
    return offset.to(dtype), coeff.to(dtype)


def gaussian_rbf(d: torch.Tensor, offset: torch.Tensor, coeff: torch.Tensor,
                 cut: Cutoff) -> torch.Tensor:
    """GaussianBasis.forward (gaussian.py:98-102)."""
    d = d.unsqueeze(-1)
    return torch.exp(coeff * torch.pow(d - offset, 2)) * cut(d)


def expnormal_params(lo: float, hi: float, num_rbf: int, dtype=torch.float32):
    """ExpNormalBasis._initial_params (mlcg/nn/radial_basis/exp_normal.py:80-94):
    means = linspace(exp(lo - hi), 1, K), betas = (2 / K (1 - exp(lo - hi)))^-2."""
    start = torch.exp(torch.scalar_tensor(-hi + lo))
    means = torch.linspace(start, 1, num_rbf)
    betas = torch.tensor([(2 / num_rbf * (1 - start)) ** -2] * num_rbf)
    return means.to(dtype), betas.to(dtype)


def expnormal_alpha(lo: float, hi: float) -> float:
    """alpha = 5 / (hi - lo) (exp_normal.py:70)."""
    return 5.0 / (hi - lo)


def expnormal_rbf(d: torch.Tensor, means: torch.Tensor, betas: torch.Tensor, alpha: float,
                  lo: float, cut: Cutoff) -> torch.Tensor:
    """ExpNormalBasis.forward (exp_normal.py:104-124):
    C(d) exp(-beta_k (exp(alpha (lo - d)) - mu_k)^2)."""
    d = d.unsqueeze(-1)
    return cut(d) * torch.exp(-betas * (torch.exp(alpha * (-d + lo)) - means) ** 2)


def shifted_softplus(x: torch.Tensor) -> torch.Tensor:
    """softplus(x) - ln 2 (the reference defines no SSP; this build's choice)."""
    return torch.nn.functional.softplus(x) - math.log(2.0)


def activation(name: str):
    if name == "tanh":
        return torch.tanh
    if name == "ssp":
        return shifted_softplus
    raise ValueError(name)


def linear(x, w, b=None):
    y = x.matmul(w.t())
    return y if b is None else y + b


def mlp(x: torch.Tensor, layers: List[Dict[str, torch.Tensor]], act) -> torch.Tensor:
    """MLP.forward (mlcg/nn/mlp.py:41-58): [Lin, act]* then Lin."""
    for k, lay in enumerate(layers):
        x = linear(x, lay["weight"], lay.get("bias"))
        if k < len(layers) - 1:
            x = act(x)
    return x


def compute_distances(pos: torch.Tensor, mapping: torch.Tensor) -> torch.Tensor:
    """compute_distances (mlcg/geometry/internal_coordinates.py:95-100)."""
    dr = pos[mapping[1]] - pos[mapping[0]]
    return dr.norm(p=2, dim=1)


# --------------------------------------------------------------------------
# SchNet

@dataclass
class SchNetConfig:
    num_rbf: int = 50
    rbf_lo: float = 0.0
    rbf_hi: float = 20.0
    rbf_cut: str = "cosine"        # cutoff inside the GaussianBasis
    conv_cut: str = "cosine"       # cutoff applied to the filters
    conv_lo: float = 0.0
    conv_hi: float = 20.0
    act: str = "tanh"
    num_blocks: int = 3
    basis: str = "gaussian"        # "gaussian" | "expnormal"
    aggr: str = "add"              # CFConv aggregation: "add" | "mean"


BASIS_KEYS = {"gaussian": ("rbf_layer.offset", "rbf_layer.coeff"),
              "expnormal": ("rbf_layer.means", "rbf_layer.betas")}


def rbf_expand(sd, cfg: SchNetConfig, distances: torch.Tensor) -> torch.Tensor:
    rbf_cut = Cutoff(cfg.rbf_cut, cfg.rbf_lo, cfg.rbf_hi)
    if cfg.basis == "gaussian":
        return gaussian_rbf(distances, sd["rbf_layer.offset"], sd["rbf_layer.coeff"], rbf_cut)
    return expnormal_rbf(distances, sd["rbf_layer.means"], sd["rbf_layer.betas"],
                         expnormal_alpha(cfg.rbf_lo, cfg.rbf_hi), cfg.rbf_lo, rbf_cut)


def _layers(sd, prefix: str) -> List[Dict[str, torch.Tensor]]:
    out = []
    k = 0
    while f"{prefix}.layers.{k}.weight" in sd:
        lay = {"weight": sd[f"{prefix}.layers.{k}.weight"]}
        if f"{prefix}.layers.{k}.bias" in sd:
            lay["bias"] = sd[f"{prefix}.layers.{k}.bias"]
        out.append(lay)
        k += 2  # activation modules take the odd indices (mlp.py:41-49)
    return out


def aggregate(msg: torch.Tensor, index: torch.Tensor, n: int, aggr: str = "add") -> torch.Tensor:
    """PyG's scatter of the messages onto their receivers (MessagePassing with
    aggr="add" or "mean"): the sum, or the sum divided by the number of
    messages, a receiver without messages getting zero."""
    agg = torch.zeros(n, msg.shape[1], dtype=msg.dtype).index_add_(0, index, msg)
    if aggr == "mean":
        cnt = torch.bincount(index, minlength=n).clamp_min(1).to(msg.dtype)
        agg = agg / cnt.unsqueeze(1)
    elif aggr not in ("add", "sum"):
        raise ValueError(f"aggr {aggr!r}")
    return agg


def schnet_energy(sd: Dict[str, torch.Tensor], cfg: SchNetConfig, pos: torch.Tensor,
                  atom_types: torch.Tensor, batch: torch.Tensor, edge_index: torch.Tensor,
                  n_frames: int) -> torch.Tensor:
    """SchNet.forward (mlcg/nn/schnet.py:116-162) with the blocks of
    InteractionBlock.forward (229-262) and CFConv.forward/message (312-368)."""
    act = activation(cfg.act)
    conv_cut = Cutoff(cfg.conv_cut, cfg.conv_lo, cfg.conv_hi)
    x = sd["embedding_layer.weight"][atom_types]
    distances = compute_distances(pos, edge_index)
    rbf = rbf_expand(sd, cfg, distances)
    for b in range(cfg.num_blocks):
        p = f"interaction_blocks.{b}"
        # CFConv.forward (schnet.py:340-347)
        C = conv_cut(distances)
        W = mlp(rbf, _layers(sd, f"{p}.conv.filter_network"), act) * C.view(-1, 1)
        y = linear(x, sd[f"{p}.conv.lin1.weight"])
        msg = y.index_select(0, edge_index[0]) * W          # x_j * W (schnet.py:368)
        agg = aggregate(msg, edge_index[1], y.shape[0], cfg.aggr)
        h = linear(agg, sd[f"{p}.conv.lin2.weight"], sd[f"{p}.conv.lin2.bias"])
        # InteractionBlock.forward (schnet.py:259-261), residual at 152-155
        v = linear(act(h), sd[f"{p}.lin.weight"], sd[f"{p}.lin.bias"])
        x = x + v
    o = mlp(x, _layers(sd, "output_network"), act)
    energy = torch.zeros(n_frames, dtype=o.dtype).index_add_(0, batch, o.view(-1))
    return energy


def schnet_energy_forces(sd, cfg, pos, atom_types, batch, edge_index, n_frames,
                         create_graph: bool = False):
    """GradientsOut.forward (mlcg/nn/gradients.py:208-226)."""
    pos = pos.detach().requires_grad_(True)
    E = schnet_energy(sd, cfg, pos, atom_types, batch, edge_index, n_frames)
    (dE,) = torch.autograd.grad(E.sum(), pos, create_graph=create_graph)
    return E, -dE


def force_mse(forces: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    """ForceMSE.forward (mlcg/nn/losses.py:177-181), reduction='mean'."""
    return torch.nn.functional.mse_loss(forces, ref, reduction="mean")


def force_matching_grads(sd, cfg, pos, atom_types, batch, edge_index, n_frames,
                         f_ref: torch.Tensor, param_names: Optional[List[str]] = None,
                         trainable_basis: bool = False):
    """PLModel.step (mlcg/pl/model.py:113-131) + loss.backward(): the loss
    mean((F - F_ref)^2) and d loss / d theta through the create_graph graph.
    The basis parameters are among theta only when trainable_basis."""
    fixed = () if trainable_basis else BASIS_KEYS[cfg.basis]
    params = {k: v.detach().clone().requires_grad_(True) for k, v in sd.items()
              if k not in fixed}
    sd2 = dict(sd)
    sd2.update(params)
    E, F = schnet_energy_forces(sd2, cfg, pos, atom_types, batch, edge_index, n_frames,
                                create_graph=True)
    loss = force_mse(F, f_ref)
    names = param_names or list(params)
    grads = torch.autograd.grad(loss, [params[k] for k in names], allow_unused=True)
    out = {}
    for k, g in zip(names, grads):
        out[k] = torch.zeros_like(params[k]) if g is None else g
    return loss.detach(), E.detach(), F.detach(), out


def force_matching_grads_chunked(sd, cfg, pos, atom_types, batch, edge_index, n_frames,
                                 f_ref: torch.Tensor, frames_per_chunk: int = 32,
                                 trainable_basis: bool = False):
    """force_matching_grads over a large batch, evaluated frame chunk by
    frame chunk to bound the memory of the create_graph graph.  Frames share
    no edges (neighbor_list.py:89-91), so energies and forces are per chunk,
    and with loss = sum_c SSE_c / (3 N) the parameter gradient is
    sum_c grad(mean_c) * N_c / N (mean_c = SSE_c / (3 N_c)).  `batch` must be
    sorted and `edge_index` grouped by frame (any edge list of the batch)."""
    N = pos.shape[0]
    counts = torch.bincount(batch, minlength=n_frames)
    ptr = torch.zeros(n_frames + 1, dtype=torch.long)
    ptr[1:] = torch.cumsum(counts, 0)
    E_all, F_all, grads, sse = [], [], None, 0.0
    for f0 in range(0, n_frames, frames_per_chunk):
        f1 = min(n_frames, f0 + frames_per_chunk)
        n0, n1 = int(ptr[f0]), int(ptr[f1])
        sel = (edge_index[0] >= n0) & (edge_index[0] < n1)
        ei = edge_index[:, sel] - n0
        loss_c, E_c, F_c, g_c = force_matching_grads(
            sd, cfg, pos[n0:n1], atom_types[n0:n1], batch[n0:n1] - f0, ei, f1 - f0,
            f_ref[n0:n1], trainable_basis=trainable_basis)
        w = (n1 - n0) / N
        sse = sse + float(loss_c) * 3 * (n1 - n0)
        E_all.append(E_c)
        F_all.append(F_c)
        if grads is None:
            grads = {k: v * w for k, v in g_c.items()}
        else:
            for k, v in g_c.items():
                grads[k] = grads[k] + v * w
    return (torch.tensor(sse / (3 * N), dtype=pos.dtype), torch.cat(E_all), torch.cat(F_all),
            grads)


# --------------------------------------------------------------------------
# Parameter construction (independent of torch.nn module init order)

def random_state_dict(cfg: SchNetConfig, hidden: int = 128, filters: int = 128,
                      embedding_size: int = 100, out_widths=(64,), seed: int = 0,
                      dtype=torch.float32, bias_scale: float = 0.1) -> Dict[str, torch.Tensor]:
    """Xavier-uniform weights (init_xavier_uniform, mlcg/nn/_module_init.py:4-28)
    drawn from a seeded generator.  Biases get small random values instead of
    zeros so that the tests exercise every bias gradient."""
    g = torch.Generator().manual_seed(seed)

    def xavier(o, i):
        a = math.sqrt(6.0 / (i + o))
        return ((torch.rand(o, i, generator=g) * 2 - 1) * a).to(dtype)

    def bias(n):
        return ((torch.rand(n, generator=g) * 2 - 1) * bias_scale).to(dtype)

    sd = {"embedding_layer.weight": torch.randn(embedding_size, hidden, generator=g).to(dtype)}
    if cfg.basis == "gaussian":
        off, coeff = gaussian_params(cfg.rbf_lo, cfg.rbf_hi, cfg.num_rbf, dtype)
        sd["rbf_layer.offset"] = off
        sd["rbf_layer.coeff"] = coeff
    else:
        means, betas = expnormal_params(cfg.rbf_lo, cfg.rbf_hi, cfg.num_rbf, dtype)
        sd["rbf_layer.means"] = means
        sd["rbf_layer.betas"] = betas
    for b in range(cfg.num_blocks):
        p = f"interaction_blocks.{b}"
        sd[f"{p}.conv.lin1.weight"] = xavier(filters, hidden)
        sd[f"{p}.conv.lin2.weight"] = xavier(hidden, filters)
        sd[f"{p}.conv.lin2.bias"] = bias(hidden)
        sd[f"{p}.conv.filter_network.layers.0.weight"] = xavier(filters, cfg.num_rbf)
        sd[f"{p}.conv.filter_network.layers.0.bias"] = bias(filters)
        sd[f"{p}.conv.filter_network.layers.2.weight"] = xavier(filters, filters)
        sd[f"{p}.lin.weight"] = xavier(hidden, hidden)
        sd[f"{p}.lin.bias"] = bias(hidden)
    widths = [hidden] + list(out_widths) + [1]
    for k in range(len(widths) - 1):
        sd[f"output_network.layers.{2 * k}.weight"] = xavier(widths[k + 1], widths[k])
        if k < len(widths) - 2:
            sd[f"output_network.layers.{2 * k}.bias"] = bias(widths[k + 1])
    return sd


def to_dtype(sd: Dict[str, torch.Tensor], dtype) -> Dict[str, torch.Tensor]:
    return {k: v.to(dtype) for k, v in sd.items()}
