"""SchNet, InteractionBlock, CFConv and StandardSchNet with the reference's
constructor signatures and state_dict keys (mlcg/nn/schnet.py:32-475).

``SchNet.forward`` runs the fused HIP path (``_fused``) whenever the model is
made of the pieces the kernels implement (Gaussian or exp-normal basis,
trainable or not, with identity/cosine envelope, MLP filters [K, 128, 128]
without last bias, Tanh or shifted softplus).  Other compositions run module by module, still on the HIP radius
graph and the HIP CFConv gather.  Tensors on the CPU are rejected: there is
no CPU implementation in this package.
"""

from __future__ import annotations

import warnings
from typing import Final, List, Optional

import torch

from .. import ops
from .._lib import require_device
from ..data._keys import ENERGY_KEY
from ..neighbor_list.neighbor_list import atomic_data2neighbor_list, validate_neighborlist
from . import _fused
from .activations import activation_id
from .cutoff import CosineCutoff, IdentityCutoff
from .mlp import MLP, init_xavier_uniform
from .radial_basis import ExpNormalBasis, GaussianBasis


class _EdgeGather(torch.autograd.Function):
    """out[t] = sum_{e: tgt_e = t} src[src_e] * W[e] over an arbitrary edge
    list (PyG propagate with aggr="add"), on the HIP gather kernel."""

    @staticmethod
    def forward(ctx, src, W, fwd_graph, bwd_graph, edge_src, edge_tgt):
        ctx.save_for_backward(src, W)
        ctx.graphs = (fwd_graph, bwd_graph, edge_src, edge_tgt)
        return ops.cfconv_gather(src.contiguous(), W.contiguous(), fwd_graph)

    @staticmethod
    def backward(ctx, gout):
        src, W = ctx.saved_tensors
        fwd_graph, bwd_graph, edge_src, edge_tgt = ctx.graphs
        gsrc = gW = None
        if ctx.needs_input_grad[0]:
            gsrc = _EdgeGather.apply(gout.contiguous(), W, bwd_graph, fwd_graph, edge_tgt,
                                     edge_src)
        if ctx.needs_input_grad[1]:
            gW = gout.index_select(0, edge_tgt) * src.index_select(0, edge_src)
        return gsrc, gW, None, None, None, None


def _edge_csr(edge_index: torch.Tensor, num_nodes: int, by_row: int) -> ops.PairGraph:
    """Receiver CSR of an edge list grouped by edge_index[by_row] (stable, so
    edges keep their order inside a row); eid2pair holds the edge ids."""
    key = edge_index[by_row]
    order = torch.sort(key, stable=True).indices
    counts = torch.bincount(key, minlength=num_nodes)
    rowptr = torch.zeros(num_nodes + 1, dtype=torch.int32, device=key.device)
    rowptr[1:] = torch.cumsum(counts, 0).to(torch.int32)
    col = edge_index[1 - by_row].index_select(0, order).to(torch.int32).contiguous()
    eid = order.to(torch.int32).contiguous()
    return ops.PairGraph(edge_index=edge_index, rowptr=rowptr, col=col, pair_ij=None,
                         pairptr=None, eid2pair=eid, frame_ptr=rowptr.new_zeros(1).long(),
                         num_nodes=num_nodes, num_edges=edge_index.shape[1], num_pairs=0)


# PyG aggregation names of CFConv (MessagePassing(aggr=...), schnet.py:292-294)
# that the CFConv kernels implement: "add" / "sum" on the fused path, "mean"
# module by module (the HIP gather divided by each receiver's in-degree).
_AGGR = ("add", "sum", "mean")


class CFConv(torch.nn.Module):
    """Continuous-filter convolution (schnet.py:265-368).

    forward(x, edge_index, edge_weight, edge_attr): W = filter_network(edge_attr)
    * cutoff(edge_weight); out = lin2(sum_{e: edge_index[1]=i} lin1(x)[edge_index[0]] * W_e).
    """

    def __init__(self, filter_network: torch.nn.Module, cutoff: torch.nn.Module,
                 in_channels: int = 128, out_channels: int = 128, num_filters: int = 128,
                 aggr: str = "add"):
        super().__init__()
        if aggr not in _AGGR:
            raise NotImplementedError(f"aggr={aggr!r}: the CFConv kernels implement "
                                      f"{', '.join(map(repr, _AGGR))}")
        self.aggr = aggr
        self.lin1 = torch.nn.Linear(in_channels, num_filters, bias=False)
        self.lin2 = torch.nn.Linear(num_filters, out_channels)
        self.filter_network = filter_network
        self.cutoff = cutoff
        self.reset_parameters()

    def reset_parameters(self):
        self.filter_network.reset_parameters()
        init_xavier_uniform(self.lin1)
        init_xavier_uniform(self.lin2)

    def forward(self, x, edge_index, edge_weight, edge_attr):
        require_device(x, edge_index)
        C = self.cutoff(edge_weight)
        W = self.filter_network(edge_attr) * C.view(-1, 1)
        y = self.lin1(x)
        n = x.shape[0]
        fwd = _edge_csr(edge_index, n, by_row=1)
        bwd = _edge_csr(edge_index, n, by_row=0)
        # float64 models (moved to double) gather in double, others in float32
        dt = torch.float64 if y.dtype == torch.float64 else torch.float32
        agg = _EdgeGather.apply(y.to(dt), W.to(dt), fwd, bwd, edge_index[0], edge_index[1])
        if self.aggr == "mean":
            # PyG's mean aggregation: the sum over a receiver's messages divided
            # by their number, zero for a receiver without any
            deg = (fwd.rowptr[1:] - fwd.rowptr[:-1]).clamp_min(1).to(agg.dtype)
            agg = agg / deg.unsqueeze(1)
        return self.lin2(agg)


class InteractionBlock(torch.nn.Module):
    """x -> lin(act(conv(x, ...))) (schnet.py:195-262)."""

    def __init__(self, cfconv_layer: torch.nn.Module, hidden_channels: int = 128,
                 activation: torch.nn.Module = torch.nn.Tanh()):
        super().__init__()
        self.conv = cfconv_layer
        self.activation = activation
        self.lin = torch.nn.Linear(hidden_channels, hidden_channels)
        self.reset_parameters()

    def reset_parameters(self):
        self.conv.reset_parameters()
        init_xavier_uniform(self.lin)

    def forward(self, x, edge_index, edge_weight, edge_attr, *args):
        x = self.conv(x, edge_index, edge_weight, edge_attr)
        x = self.activation(x)
        return self.lin(x)


_NL_METHODS = ("torch", "custom_kernel", "hip")


def _basis_tensors(rbf):
    """(centers, widths) of a basis the filter kernels evaluate -- Gaussian
    (offset [K], coeff []) or exp-normal (means [K], betas [K]) -- else None."""
    if isinstance(rbf, GaussianBasis):
        return rbf.offset, rbf.coeff
    if isinstance(rbf, ExpNormalBasis):
        return rbf.means, rbf.betas
    return None


class SchNet(torch.nn.Module):
    """SchNet energy model (schnet.py:32-192)."""

    name: Final[str] = "SchNet"

    def __init__(self, embedding_layer: torch.nn.Module, interaction_blocks,
                 rbf_layer: torch.nn.Module, output_network: torch.nn.Module,
                 self_interaction: bool = False, max_num_neighbors: int = 1000,
                 nls_distance_method: str = "torch"):
        super().__init__()
        self.embedding_layer = embedding_layer
        self.rbf_layer = rbf_layer
        self.max_num_neighbors = max_num_neighbors
        if self_interaction:
            raise NotImplementedError(
                "The option `self_interaction` did not have function due to a bug. It only "
                "exists for compatibility and should stay `False`.")
        self.self_interaction = self_interaction
        if isinstance(interaction_blocks, list):
            self.interaction_blocks = torch.nn.Sequential(*interaction_blocks)
        elif isinstance(interaction_blocks, InteractionBlock):
            self.interaction_blocks = torch.nn.Sequential(interaction_blocks)
        else:
            raise RuntimeError("interaction_blocks must be a single InteractionBlock or a "
                               "list of InteractionBlocks.")
        if nls_distance_method not in _NL_METHODS:
            raise ValueError(
                f"Method {nls_distance_method} not supported for nls-distance computation "
                f"(available: {_NL_METHODS}; all use the HIP radius graph)")
        self.nls_distance_method = nls_distance_method
        self.output_network = output_network
        # fp16 operands (fp32 accumulation) for the filter-network matmuls
        self.fp16_filters = False
        # fp32 filter forward on the fp32 MFMA throughout instead of the
        # default split-fp16 products (about 22 significant bits per operand)
        self.strict_fp32_filters = False
        # fixed edge capacity of the radius graph (None: sized exactly with
        # one host sync per call; an int: no sync, as needed inside a captured
        # graph -- the caller then checks last_graph.flags)
        self.graph_capacity: Optional[int] = None
        self.last_graph: Optional[ops.PairGraph] = None
        self.reset_parameters()

    def reset_parameters(self):
        self.embedding_layer.reset_parameters()
        self.rbf_layer.reset_parameters()
        for block in self.interaction_blocks:
            block.reset_parameters()
        self.output_network.reset_parameters()

    # ------------------------------------------------------------------
    def neighbor_list(self, data, rcut: float, max_num_neighbors: int = 1000) -> dict:
        return {SchNet.name: atomic_data2neighbor_list(
            data, rcut, self_interaction=False, max_num_neighbors=max_num_neighbors,
            nls_distance_method=self.nls_distance_method)}

    def is_nl_compatible(self, nl) -> bool:
        # the reference reads a non-existent self.cutoff here (schnet.py:170);
        # the rbf layer's upper cutoff is the cutoff the neighbour list needs
        return (validate_neighborlist(nl) and nl["order"] == 2
                and nl["self_interaction"] is False
                and nl["rcut"] == self.rbf_layer.cutoff.cutoff_upper)

    # ------------------------------------------------------------------
    def fused_spec(self) -> Optional[_fused.FusedSpec]:
        """The kernel description of this model, or None if some piece has no
        kernel (then forward runs module by module).  Cached, so that the
        fused path can run inside a stream capture: the spec holds the basis
        tensors themselves (float32 views of the module's own parameters or
        buffers), so in-place updates reach the kernels without a rebuild."""
        rbf = self.rbf_layer
        bt = _basis_tensors(rbf)
        key = (bool(self.fp16_filters), bool(self.strict_fp32_filters), type(rbf),
               len(self.interaction_blocks),
               bool(getattr(rbf, "trainable", False)), self._param_dtype())
        if bt is not None:
            # a float32 contiguous tensor is used in place; anything else is
            # converted, and the conversion is redone when the source changes
            key += tuple((t.data_ptr(), t.dtype, t.is_contiguous(),
                          None if t.dtype == torch.float32 and t.is_contiguous() else t._version)
                         for t in bt)
        cached = self.__dict__.get("_spec_cache")
        if cached is not None and cached[0] == key:
            return cached[1]
        spec = self._build_fused_spec()
        self.__dict__["_spec_cache"] = (key, spec)
        return spec

    def _param_dtype(self):
        w = getattr(self.embedding_layer, "weight", None)
        return None if w is None else w.dtype

    def _build_fused_spec(self) -> Optional[_fused.FusedSpec]:
        rbf = self.rbf_layer
        if self._param_dtype() != torch.float32:
            return None  # a model moved to double runs module by module in float64
        bt = _basis_tensors(rbf)
        if bt is None or bt[1].numel() != (bt[0].numel() if isinstance(rbf, ExpNormalBasis)
                                           else 1):
            return None
        if not isinstance(self.embedding_layer, torch.nn.Embedding):
            return None
        rc = rbf.cutoff
        if not isinstance(rc, (IdentityCutoff, CosineCutoff)):
            return None
        conv_cut = None
        filt_act = block_act = None
        for blk in self.interaction_blocks:
            if not isinstance(blk, InteractionBlock) or not isinstance(blk.conv, CFConv):
                return None
            if blk.conv.aggr not in ("add", "sum"):
                return None
            fn = blk.conv.filter_network
            if not isinstance(fn, MLP):
                return None
            lins = fn.linears()
            acts = fn.activations()
            if (len(lins) != 2 or len(acts) != 1 or lins[1].bias is not None
                    or lins[0].bias is None or lins[0].out_features != ops.NUM_FILTERS
                    or lins[1].out_features != ops.NUM_FILTERS
                    or lins[0].in_features != bt[0].numel()):
                return None
            c = blk.conv.cutoff
            if not isinstance(c, (IdentityCutoff, CosineCutoff)):
                return None
            key = (type(c), c.cutoff_lower, c.cutoff_upper)
            if conv_cut is None:
                conv_cut = key
            elif conv_cut != key:
                return None
            fa, ba = activation_id(acts[0]), activation_id(blk.activation)
            if fa is None or ba is None:
                return None
            if filt_act is None:
                filt_act, block_act = fa, ba
            elif (filt_act, block_act) != (fa, ba):
                return None
        out_acts = self.output_network.activations() if isinstance(
            self.output_network, MLP) else None
        if out_acts is None:
            return None
        oa = {activation_id(a) for a in out_acts}
        if None in oa or len(oa) > 1:
            return None
        out_act = oa.pop() if oa else 0
        c0 = self.interaction_blocks[0].conv.cutoff
        centers, widths = (t.detach().float().reshape(-1).contiguous() for t in bt)
        filt = ops.FilterSpec(
            centers=centers, widths=widths, num_rbf=centers.numel(),
            basis=ops.BASIS_EXPNORMAL if isinstance(rbf, ExpNormalBasis) else ops.BASIS_GAUSSIAN,
            alpha=float(getattr(rbf, "alpha", 0.0)),
            rbf_cut_kind=rc.kind_id, rbf_lo=float(rc.cutoff_lower),
            rbf_hi=float(min(rc.cutoff_upper, 3.0e38)),
            conv_cut_kind=c0.kind_id, conv_lo=float(c0.cutoff_lower),
            conv_hi=float(min(c0.cutoff_upper, 3.0e38)), act=filt_act)
        return _fused.FusedSpec(
            filt=filt, filter_act=filt_act, block_act=block_act, out_act=out_act,
            num_blocks=len(self.interaction_blocks),
            out_has_bias=[lin.bias is not None for lin in self.output_network.linears()],
            f16=bool(self.fp16_filters), basis_trainable=bool(rbf.trainable),
            strict_fp32=bool(self.strict_fp32_filters))

    def fused_params(self) -> _fused.Params:
        blocks = []
        for blk in self.interaction_blocks:
            l0, l2 = blk.conv.filter_network.linears()
            blocks.append(_fused.BlockParams(
                W1=l0.weight, b1=l0.bias, W2=l2.weight, A1=blk.conv.lin1.weight,
                A2=blk.conv.lin2.weight, c2=blk.conv.lin2.bias, A3=blk.lin.weight,
                c3=blk.lin.bias))
        lins = self.output_network.linears()
        rbf = self.rbf_layer
        basis = list(_basis_tensors(rbf)) if getattr(rbf, "trainable", False) else []
        return _fused.Params(emb=self.embedding_layer.weight, blocks=blocks,
                             out_w=[lin.weight for lin in lins],
                             out_b=[lin.bias for lin in lins], basis=basis)

    def build_graph(self, data) -> ops.PairGraph:
        """Radius graph with the receiver CSR and pair map (HIP kernels)."""
        require_device(data.pos)
        n = data.pos.shape[0]
        batch = data.batch if "batch" in data else torch.zeros(
            n, dtype=torch.long, device=data.pos.device)
        n_frames = int(data.n_atoms.numel()) if "n_atoms" in data else None
        g = ops.radius_graph(data.pos.detach(), float(self.rbf_layer.cutoff.cutoff_upper),
                             batch=batch, loop=False, max_num_neighbors=self.max_num_neighbors,
                             with_pairs=True, n_frames=n_frames,
                             capacity=self.graph_capacity)
        self.last_graph = g
        return g

    # ------------------------------------------------------------------
    # The fused path launches HIP kernels through ctypes: torch.compile runs
    # it as an opaque call (a graph break), the compiled code around it
    # unchanged.
    @torch.compiler.disable
    def forward(self, data):
        spec = self.fused_spec()
        if spec is None:
            return self._forward_modular(data)
        require_device(data.pos)
        graph = self.build_graph(data)
        P = self.fused_params()
        pos = data.pos
        batch = data.batch if "batch" in data else torch.zeros(
            pos.shape[0], dtype=torch.long, device=pos.device)
        E = _fused.Energy.apply(spec, data.atom_types, batch, graph, pos.float(), *P.flat())
        data.out[self.name] = {ENERGY_KEY: E}
        return data

    @torch.compiler.disable
    def energy_forces(self, data, create_graph: bool):
        """Fused energy and forces (used by GradientsOut)."""
        spec = self.fused_spec()
        require_device(data.pos)
        graph = self.build_graph(data)
        P = self.fused_params()
        batch = data.batch if "batch" in data else torch.zeros(
            data.pos.shape[0], dtype=torch.long, device=data.pos.device)
        return _fused.EnergyForces.apply(spec, data.pos.detach().float(), data.atom_types,
                                         batch, graph, bool(create_graph), *P.flat())

    def _forward_modular(self, data):
        require_device(data.pos)
        x = self.embedding_layer(data.atom_types)
        nl = self.neighbor_list(data, self.rbf_layer.cutoff.cutoff_upper,
                                self.max_num_neighbors)[self.name]
        edge_index = nl["index_mapping"]
        dr = data.pos[edge_index[1]] - data.pos[edge_index[0]]
        distances = dr.norm(p=2, dim=1)
        rbf_expansion = self.rbf_layer(distances)
        num_batch = data.batch[-1] + 1
        for block in self.interaction_blocks:
            x = x + block(x, edge_index, distances, rbf_expansion, num_batch, data.batch)
        energy = self.output_network(x, data).view(-1)
        frame_ptr = ops.frame_ptr_from_batch(data.batch, int(num_batch))
        energy = _SegmentSum.apply(energy, frame_ptr, data.batch)
        data.out[self.name] = {ENERGY_KEY: energy}
        return data


class _SegmentSum(torch.autograd.Function):
    @staticmethod
    def forward(ctx, values, frame_ptr, batch):
        ctx.batch = batch
        return ops.segment_sum(values if values.dtype == torch.float64 else values.float(),
                               frame_ptr)

    @staticmethod
    def backward(ctx, g):
        return g.index_select(0, ctx.batch), None, None


class StandardSchNet(SchNet):
    """SchNet built from widths (schnet.py:371-475); identical construction
    order, module tree and state_dict keys."""

    def __init__(self, rbf_layer: torch.nn.Module, cutoff: torch.nn.Module,
                 output_hidden_layer_widths: List[int], hidden_channels: int = 128,
                 embedding_size: int = 100, num_filters: int = 128, num_interactions: int = 3,
                 activation: torch.nn.Module = torch.nn.Tanh(), max_num_neighbors: int = 1000,
                 aggr: str = "add", nls_distance_method: str = "torch"):
        if num_interactions < 1:
            raise ValueError("At least one interaction block must be specified")
        if cutoff.cutoff_lower != rbf_layer.cutoff.cutoff_lower:
            warnings.warn(
                "Cutoff function lower cutoff, {}, and radial basis function  lower cutoff, "
                "{}, do not match.".format(cutoff.cutoff_lower, rbf_layer.cutoff.cutoff_lower))
        if cutoff.cutoff_upper != rbf_layer.cutoff.cutoff_upper:
            warnings.warn(
                "Cutoff function upper cutoff, {}, and radial basis function  upper cutoff, "
                "{}, do not match.".format(cutoff.cutoff_upper, rbf_layer.cutoff.cutoff_upper))
        embedding_layer = torch.nn.Embedding(embedding_size, hidden_channels)
        interaction_blocks = []
        for _ in range(num_interactions):
            filter_network = MLP(layer_widths=[rbf_layer.num_rbf, num_filters, num_filters],
                                 activation_func=activation, last_bias=False)
            cfconv = CFConv(filter_network, cutoff=cutoff, num_filters=num_filters,
                            in_channels=hidden_channels, out_channels=hidden_channels,
                            aggr=aggr)
            interaction_blocks.append(InteractionBlock(cfconv, hidden_channels, activation))
        output_layer_widths = [hidden_channels] + output_hidden_layer_widths + [1]
        output_network = MLP(output_layer_widths, activation_func=activation, last_bias=False)
        super().__init__(embedding_layer, interaction_blocks, rbf_layer, output_network,
                         max_num_neighbors=max_num_neighbors,
                         nls_distance_method=nls_distance_method)
