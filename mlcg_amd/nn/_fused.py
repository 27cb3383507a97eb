"""Fused SchNet energy / force / force-matching evaluation on the HIP kernels.

This is the hot path of the package.  Edge work (filter network, CFConv
gather/scatter, their backward, tangent and second-order reverse, the pair ->
node force scatter) and node work (the [N, H] x [H, H] linears with their
bias / residual / activation epilogues, the output network) run in the gfx950
kernels of ``libmlcg_hip.so``, all on torch's current stream.

Math (per interaction block, activation s = act(z)):
    y = x A1^T ;  agg_i = sum_j y_j * W_ij ;  z = agg A2^T + c2 ;  v = s A3^T + c3 ;
    x <- x + v ;  o = MLP_out(x) ;  E_b = sum_{n in b} o_n
with W_ij = filter(d_ij) evaluated per unordered pair, and Wd = dW/dd.

* reverse1 (forces): the usual reverse sweep, plus per pair
  dbar_p = sum_blocks <Wd_p, gagg_i y_j + gagg_j y_i>, and
  F_i = sum_j dbar_p (pos_j - pos_i) / d_p.
* tangent: forward-mode derivative along a position direction u
  (ddot_p = rhat_p . (u_j - u_i), Wdot = Wd ddot).
* reverse2: reverse sweep of (primal, tangent) for d/dtheta of
  sum_n tw_n odot_n + pw_n o_n.  The tangent adjoints equal the reverse1
  adjoints when reverse1 was seeded with tw, so only the primal adjoints are
  new.  This is the hand-derived double backward of the force-matching loss
  L(F): with u = -dL/dF it gives dL/dtheta, replacing the autograd replay of
  create_graph=True (mlcg/nn/gradients.py:216-222, mlcg/pl/model.py:113-131).
* trainable basis parameters theta_b: the filter backward also emits the
  first-layer pair adjoints abar = dL/da and adbar = dL/da' (a = W1 g + b1,
  a' = W1 g'), and dL/dtheta_b = sum_p (W1^T abar_p) . dg/dtheta_b
  + (W1^T adbar_p) . dg'/dtheta_b, summed over blocks.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace
from typing import List, Optional, Tuple

import os

import torch

from .. import ops
from .activations import ACT_TANH, act_derivs, act_value


@dataclass
class BlockParams:
    W1: torch.Tensor  # filter layer 0 weight [F, K]
    b1: torch.Tensor  # filter layer 0 bias [F]
    W2: torch.Tensor  # filter layer 2 weight [F, F]
    A1: torch.Tensor  # conv.lin1.weight [F, H]
    A2: torch.Tensor  # conv.lin2.weight [H, F]
    c2: torch.Tensor  # conv.lin2.bias [H]
    A3: torch.Tensor  # lin.weight [H, H]
    c3: torch.Tensor  # lin.bias [H]

    def tensors(self) -> List[torch.Tensor]:
        return [self.W1, self.b1, self.W2, self.A1, self.A2, self.c2, self.A3, self.c3]


@dataclass
class FusedSpec:
    """Static (non-tensor) description of a fusable SchNet."""

    filt: ops.FilterSpec
    filter_act: int
    block_act: int
    out_act: int
    num_blocks: int
    out_has_bias: List[bool]  # per output linear
    f16: bool = False
    basis_trainable: bool = False  # Params.basis carries (centers, widths)
    strict_fp32: bool = False  # filter forward on the fp32 MFMA throughout


@dataclass
class Params:
    emb: torch.Tensor
    blocks: List[BlockParams]
    out_w: List[torch.Tensor]
    out_b: List[Optional[torch.Tensor]]
    basis: List[torch.Tensor] = field(default_factory=list)  # trainable (centers, widths)

    def flat(self) -> List[torch.Tensor]:
        out = [self.emb]
        for b in self.blocks:
            out += b.tensors()
        for w, b in zip(self.out_w, self.out_b):
            out.append(w)
            if b is not None:
                out.append(b)
        return out + list(self.basis)

    @staticmethod
    def unflat(spec: FusedSpec, flat: List[torch.Tensor]) -> "Params":
        it = iter(flat)
        emb = next(it)
        blocks = [BlockParams(*[next(it) for _ in range(8)]) for _ in range(spec.num_blocks)]
        out_w, out_b = [], []
        for has_b in spec.out_has_bias:
            out_w.append(next(it))
            out_b.append(next(it) if has_b else None)
        basis = [next(it), next(it)] if spec.basis_trainable else []
        return Params(emb, blocks, out_w, out_b, basis)


def filter_spec(spec: FusedSpec, P: Params) -> ops.FilterSpec:
    """The filter description with the basis tensors of this call (the
    trainable parameters when the basis is trained)."""
    if not spec.basis_trainable:
        return spec.filt
    c, w = (t.detach().float().reshape(-1).contiguous() for t in P.basis)
    return replace(spec.filt, centers=c, widths=w)


@dataclass
class State:
    """Activations saved by forward / reverse1 / tangent."""

    pos: torch.Tensor
    types: torch.Tensor
    graph: ops.PairGraph
    filt: Optional[ops.FilterSpec] = None
    dist: Optional[torch.Tensor] = None
    W: List[torch.Tensor] = field(default_factory=list)
    Wd: List[torch.Tensor] = field(default_factory=list)
    x: List[torch.Tensor] = field(default_factory=list)    # block inputs
    y: List[torch.Tensor] = field(default_factory=list)
    agg: List[torch.Tensor] = field(default_factory=list)
    z: List[torch.Tensor] = field(default_factory=list)
    s: List[torch.Tensor] = field(default_factory=list)
    xL: Optional[torch.Tensor] = None
    # split images of the block weights, {(block, "A1" | "A2" | "A3", transpose)}
    wimg: Optional[dict] = None
    oh: List[torch.Tensor] = field(default_factory=list)   # output-MLP layer inputs
    oz: List[torch.Tensor] = field(default_factory=list)   # output-MLP pre-activations
    os_: List[torch.Tensor] = field(default_factory=list)  # output-MLP activations
    o: Optional[torch.Tensor] = None
    # reverse1
    xbar_out: List[torch.Tensor] = field(default_factory=list)
    sbar1: List[torch.Tensor] = field(default_factory=list)
    zbar1: List[torch.Tensor] = field(default_factory=list)
    gagg1: List[torch.Tensor] = field(default_factory=list)
    ybar1: List[torch.Tensor] = field(default_factory=list)
    # tangent
    ddot: Optional[torch.Tensor] = None
    xdot_in: List[Optional[torch.Tensor]] = field(default_factory=list)
    ydot: List[Optional[torch.Tensor]] = field(default_factory=list)
    aggdot: List[torch.Tensor] = field(default_factory=list)
    zdot: List[torch.Tensor] = field(default_factory=list)
    sdot: List[torch.Tensor] = field(default_factory=list)
    ohdot: List[torch.Tensor] = field(default_factory=list)
    ozdot: List[torch.Tensor] = field(default_factory=list)
    odot: Optional[torch.Tensor] = None
    # fused output network
    xdotL: Optional[torch.Tensor] = None      # tangent of the last block output
    out_seed: Optional[torch.Tensor] = None   # reverse seed the forward already applied
    out_xbar: Optional[torch.Tensor] = None   # ... and the adjoint it produced


def _out_fused(P: "Params") -> bool:
    """True when the output network is MLP([128, HH, 1]) with HH in the
    kernel's set (StandardSchNet's [64] default shape)."""
    return (len(P.out_w) == 2 and P.out_w[1].shape[0] == 1
            and P.out_w[0].shape[1] == ops.NUM_FILTERS
            and P.out_w[0].shape[0] in ops.OUT_HIDDEN
            and P.out_w[1].shape[1] == P.out_w[0].shape[0])


def _lin(x, w, b=None):
    return torch.addmm(b, x, w.t()) if b is not None else x.mm(w.t())


# Node linears with their elementwise neighbours fused (mlcg_node_gemm); the
# unfused forms serve hidden widths the kernel does not tile.

def _lin_act(x, A, c, act, want_z):
    """(z, s) = (x A^T + c, act(z)); z is None when not wanted."""
    if ops._node_gemm_ok(x, A):
        return ops.node_gemm(x, A, bias=c, epilogue=ops.NODE_ACT, act=act, want_out0=want_z)
    z = ops.node_linear(x, A, bias=c)
    return z, act_value(z, act)


def _lin_dact(x, A, z, s, act, transpose):
    """(y, y * act'(z)) with y = x A^T (x A with transpose)."""
    if ops._node_gemm_ok(x, A):
        return ops.node_gemm(x, A, transpose=transpose, epilogue=ops.NODE_DACT, act=act, z=z,
                             s=s)
    y = ops.node_linear(x, A, transpose=transpose)
    d1, _ = act_derivs(z, s, act)
    return y, y * d1


def _lin_dact2(x, A, z, s, act, e, f):
    """(x A) * act'(z) [+ e * act''(z) * f]."""
    if ops._node_gemm_ok(x, A):
        return ops.node_gemm(x, A, transpose=True, epilogue=ops.NODE_DACT2, act=act, z=z, s=s,
                             e=e, f=f)[0]
    y = ops.node_linear(x, A, transpose=True)
    d1, d2 = act_derivs(z, s, act)
    v = y * d1
    return v if e is None else v + e * d2 * f


# Consecutive node linears in one kernel (mlcg_node_gemm2): the first
# product's activation output feeds the second without a round trip through
# memory; results are bit-identical to the two separate calls.

def _gemm2_ok(x, A, B):
    return ops._node_gemm_ok(x, A) and ops._node_gemm_ok(x, B)


def _lin_act_lin(x, A, c, act, want_z, B, cb, residual, imgs=(None, None)):
    """(z, s, s B^T + cb + residual) with (z, s) = _lin_act(x, A, c, act);
    imgs: the split images of A and B for this orientation (or None)."""
    if _gemm2_ok(x, A, B):
        return ops.node_gemm2(x, A, B, bias=c, epilogue=ops.NODE_ACT, act=act,
                              want_out0=want_z, bias2=cb, residual2=residual,
                              w_image=imgs[0], w2_image=imgs[1])
    z, s = _lin_act(x, A, c, act, want_z)
    return z, s, ops.node_linear(s, B, bias=cb, residual=residual)


def _lin_dact_lin(x, A, z, s, act, transpose, B, residual=None, imgs=(None, None),
                  keep: bool = True):
    """(y, v, v B^T [+ residual]) (v B with transpose), (y, v) = _lin_dact(...);
    keep=False: y and v may be None (not written) when the fused kernel runs."""
    if _gemm2_ok(x, A, B):
        return ops.node_gemm2(x, A, B, transpose=transpose, epilogue=ops.NODE_DACT, act=act,
                              z=z, s=s, residual2=residual, w_image=imgs[0],
                              w2_image=imgs[1], want_out0=keep, want_out1=keep)
    y, v = _lin_dact(x, A, z, s, act, transpose)
    return y, v, ops.node_linear(v, B, transpose=transpose, residual=residual)


def _lin_dact2_lin(x, A, z, s, act, e, f, B, imgs=(None, None)):
    """(v, v B) with v = _lin_dact2(x, A, z, s, act, e, f)."""
    if _gemm2_ok(x, A, B):
        v, _, out = ops.node_gemm2(x, A, B, transpose=True, epilogue=ops.NODE_DACT2, act=act,
                                   z=z, s=s, e=e, f=f, w_image=imgs[0], w2_image=imgs[1])
        return v, out
    v = _lin_dact2(x, A, z, s, act, e, f)
    return v, ops.node_linear(v, B, transpose=True)


# Filter forwards of blocks 1.. on the side stream (MLCG_FILTER_AHEAD=0 keeps
# them in block order on the caller's stream).
_FILTER_AHEAD = os.environ.get("MLCG_FILTER_AHEAD", "1") != "0"


def _filters_ahead(spec: FusedSpec, P: Params, pos: torch.Tensor, graph: ops.PairGraph,
                   filt) -> dict:
    """Issues the filter forwards of blocks 1.. on the side stream at the start
    of the forward: they depend only on the pair distances and the block's
    filter weights, not on node features, so they run beside block 0's node
    linears and gathers (memory-bound work that leaves VGPRs and LDS free on
    each CU).  Returns {k: (W, Wd, event)}; the caller's stream waits on the
    event before block k's gather.  The outputs are allocated on the caller's
    stream, which alone uses them afterwards."""
    if not (_FILTER_AHEAD and pos.is_cuda and len(P.blocks) > 1):
        return {}
    main = torch.cuda.current_stream(pos.device)
    key = (pos.device.index, main.cuda_stream)
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=pos.device)
    side = _SIDE_STREAMS[key]
    cap = graph.pair_capacity
    dt = torch.float16 if spec.f16 else torch.float32
    outs = {k: (torch.empty(cap, ops.NUM_FILTERS, dtype=dt, device=pos.device),
                torch.empty(cap, ops.NUM_FILTERS, dtype=dt, device=pos.device))
            for k in range(1, len(P.blocks))}
    side.wait_stream(main)
    ahead = {}
    with torch.cuda.stream(side):
        for k in range(1, len(P.blocks)):
            bp = P.blocks[k]
            W, Wd, _ = ops.filter_fwd(pos, graph, filt, bp.W1, bp.b1, bp.W2, f16=spec.f16,
                                      want_dist=False, strict_fp32=spec.strict_fp32,
                                      out=outs[k])
            ev = torch.cuda.Event()
            ev.record(side)
            ahead[k] = (W, Wd, ev)
    return ahead


# Split images of the block weights made once per forward (MLCG_NODE_IMAGES=0
# lets every node GEMM launch split its weights itself; same results).
_NODE_IMAGES = os.environ.get("MLCG_NODE_IMAGES", "1") != "0"
_IMAGE_NAMES = ("A1", "A2", "A3")


def _weight_images(P: Params, x: torch.Tensor, transposed: bool) -> Optional[dict]:
    """{(block, name, transpose): image} of every block weight A1, A2, A3 in
    the orientations the sweeps use (x A^T forward and tangent; x A in the
    backward sweeps, when transposed), made in one launch from the weights
    as they are now; None when a weight is not a [128, 128] fp32 tensor on
    the GPU (those products split in the kernel or use the library GEMM)."""
    if not (_NODE_IMAGES and x.is_cuda and P.blocks):
        return None
    if not all(ops._node_gemm_ok(x, getattr(bp, n)) for bp in P.blocks for n in _IMAGE_NAMES):
        return None
    keys = [(k, n, t) for k in range(len(P.blocks)) for n in _IMAGE_NAMES
            for t in ((False, True) if transposed else (False,))]
    imgs = ops.node_weight_images([getattr(P.blocks[k], n) for k, n, _ in keys],
                                  [t for _, _, t in keys])
    return {key: imgs[i] for i, key in enumerate(keys)}


def _wi(st: "State", k: int, name: str, transpose: bool) -> Optional[torch.Tensor]:
    return None if st.wimg is None else st.wimg.get((k, name, transpose))


def forward(spec: FusedSpec, P: Params, pos: torch.Tensor, types: torch.Tensor,
            graph: ops.PairGraph, save: bool = True,
            rev_seed: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, State]:
    """Energies [B] and the saved state.  With rev_seed, the output network's
    kernel also forms the adjoint a following reverse1(seed=rev_seed) starts
    from."""
    st = State(pos=pos, types=types, graph=graph, filt=filter_spec(spec, P))
    # the lookup goes first: the side stream's filter forwards then start
    # with the first block's node products already queued behind it
    if (P.emb.dim() == 2 and P.emb.shape[1] == ops.NUM_FILTERS
            and P.emb.dtype == torch.float32 and types.dtype == torch.int64):
        x = ops.embedding_gather(P.emb.detach(), types)
    else:
        x = P.emb.index_select(0, types)
    # the weight images before the side stream's filter forwards, which would
    # otherwise hold every CU while this short launch waits for one
    st.wimg = _weight_images(P, x, transposed=save)
    ahead = _filters_ahead(spec, P, pos, graph, st.filt)
    for k, bp in enumerate(P.blocks):
        if k in ahead:
            W, Wd, done = ahead[k]
            dist = None
        else:
            W, Wd, dist = ops.filter_fwd(pos, graph, st.filt, bp.W1, bp.b1, bp.W2,
                                         f16=spec.f16, want_dist=(k == 0),
                                         strict_fp32=spec.strict_fp32)
            done = None
        if k == 0:
            st.dist = dist
        y = ops.node_linear(x, bp.A1, w_image=_wi(st, k, "A1", False))
        if done is not None:
            torch.cuda.current_stream(pos.device).wait_event(done)
        agg = ops.cfconv_gather(y, W, graph)
        # z itself is only read back by the shifted-softplus derivatives;
        # x_next = x + lin(act(z))
        z, s, x_next = _lin_act_lin(agg, bp.A2, bp.c2, spec.block_act,
                                    save and spec.block_act != ACT_TANH, bp.A3, bp.c3, x,
                                    imgs=(_wi(st, k, "A2", False), _wi(st, k, "A3", False)))
        st.W.append(W)
        st.Wd.append(Wd)
        if save:
            st.x.append(x)
            st.y.append(y)
            st.agg.append(agg)
            st.z.append(z)
            st.s.append(s)
        x = x_next
    st.xL = x
    if _out_fused(P):
        o, oz, os_, xbar = ops.out_forward(x, P.out_w[0], P.out_b[0], P.out_w[1], P.out_b[1],
                                           spec.out_act, seed=rev_seed,
                                           reverse=rev_seed is not None, save=save)
        st.oz, st.os_, st.o = [oz], [os_], o
        if rev_seed is not None:
            st.out_seed, st.out_xbar = rev_seed, xbar
        return ops.segment_sum(o, graph.frame_ptr), st
    h = x
    n_lin = len(P.out_w)
    for k in range(n_lin):
        st.oh.append(h)
        zz = _lin(h, P.out_w[k], P.out_b[k])
        if k < n_lin - 1:
            ss = act_value(zz, spec.out_act)
            st.oz.append(zz)
            st.os_.append(ss)
            h = ss
        else:
            h = zz
    st.o = h
    E = ops.segment_sum(h, graph.frame_ptr)
    return E, st


def reverse1(spec: FusedSpec, P: Params, st: State, seed: torch.Tensor,
             need_forces: bool = True, keep_adjoints: bool = True) -> Optional[torch.Tensor]:
    """First-order reverse seeded with d(objective)/d o_n = seed[n]; returns
    the forces -d/dpos (sum_n seed_n o_n) and saves the adjoints."""
    graph = st.graph
    n_lin = len(P.out_w)
    if _out_fused(P):
        if st.out_seed is seed:
            xbar = st.out_xbar
        else:
            xbar = ops.out_forward(st.xL, P.out_w[0], P.out_b[0], P.out_w[1], P.out_b[1],
                                   spec.out_act, seed=seed, reverse=True, want_o=False,
                                   save=False)[3]
        st.out_seed = st.out_xbar = None
    else:
        hbar = seed.view(-1, 1) * P.out_w[-1]  # [N, n_last_in]
        for k in range(n_lin - 2, -1, -1):
            d1, _ = act_derivs(st.oz[k], st.os_[k], spec.out_act)
            zbar = hbar * d1
            hbar = zbar.mm(P.out_w[k])
        xbar = hbar
    nb = len(P.blocks)
    # the last block's gather stores dbar, the others add to it
    dbar = (torch.empty if nb else torch.zeros)(graph.pair_capacity, dtype=torch.float32,
                                                 device=st.pos.device)
    st.xbar_out = [None] * nb
    st.sbar1 = [None] * nb
    st.zbar1 = [None] * nb
    st.gagg1 = [None] * nb
    st.ybar1 = [None] * nb
    for k in range(nb - 1, -1, -1):
        bp = P.blocks[k]
        # sbar, zbar feed only the second sweep: without keep_adjoints (energies
        # and forces alone) the fused kernel does not write them
        sbar, zbar, gagg = _lin_dact_lin(xbar, bp.A3, st.z[k], st.s[k], spec.block_act, True,
                                         bp.A2, imgs=(_wi(st, k, "A3", True),
                                                      _wi(st, k, "A2", True)),
                                         keep=keep_adjoints)
        # the first block's input is the embedding, which does not depend on
        # the positions: its ybar (and the adjoint of its input) enter neither
        # the forces nor the second sweep (whose first block has no input
        # tangent), so only its distance adjoints are formed
        ybar = ops.cfconv_gather_bwd(gagg, st.y[k], st.W[k], st.Wd[k], graph, dbar,
                                     accumulate=(k != nb - 1), want_ybar=(k != 0))
        st.xbar_out[k] = xbar
        st.sbar1[k] = sbar
        st.zbar1[k] = zbar
        st.gagg1[k] = gagg
        st.ybar1[k] = ybar
        if k != 0:
            xbar = ops.node_linear(ybar, bp.A1, transpose=True, residual=xbar,
                                   w_image=_wi(st, k, "A1", True))
    if not need_forces:
        return None
    return ops.pair_forces(st.pos, st.dist, dbar, graph)


def tangent(spec: FusedSpec, P: Params, st: State, u: torch.Tensor,
            scale: float = 1.0) -> None:
    """Forward-mode sweep along position direction scale * u.  The output
    network's tangent odot lands in st.odot here, or -- with the fused output
    network -- in the following reverse2(want_odot=True)."""
    graph = st.graph
    st.ddot = ops.pair_ddot(st.pos, st.dist, graph, u, scale)
    xdot = None
    st.xdot_in, st.ydot, st.aggdot, st.zdot, st.sdot = [], [], [], [], []
    for k, bp in enumerate(P.blocks):
        ydot = None if xdot is None else ops.node_linear(xdot, bp.A1,
                                                         w_image=_wi(st, k, "A1", False))
        aggdot = ops.cfconv_gather_tangent(ydot, st.y[k], st.W[k], st.Wd[k], st.ddot, graph)
        zdot, sdot, xdot_next = _lin_dact_lin(aggdot, bp.A2, st.z[k], st.s[k], spec.block_act,
                                              False, bp.A3, residual=xdot,
                                              imgs=(_wi(st, k, "A2", False),
                                                    _wi(st, k, "A3", False)))
        st.xdot_in.append(xdot)
        st.ydot.append(ydot)
        st.aggdot.append(aggdot)
        st.zdot.append(zdot)
        st.sdot.append(sdot)
        xdot = xdot_next
    st.xdotL = xdot
    st.odot = None
    if _out_fused(P):
        return
    hdot = xdot
    n_lin = len(P.out_w)
    st.ohdot, st.ozdot = [], []
    for k in range(n_lin):
        st.ohdot.append(hdot)
        zd = hdot.mm(P.out_w[k].t())
        if k < n_lin - 1:
            d1, _ = act_derivs(st.oz[k], st.os_[k], spec.out_act)
            st.ozdot.append(zd)
            hdot = d1 * zd
        else:
            hdot = zd
    st.odot = hdot


def _out_reverse2(spec, P, st, tw, pw, want_odot):
    """Output-network part of reverse2 as one kernel: (xbar2, g_out_w,
    g_out_b); also sets st.odot when asked."""
    tangent_on = tw is not None
    odot, xbar2, gW0, gb0, gW1, gb1 = ops.out_rev2(
        st.xL, st.xdotL if (tangent_on or want_odot) else None, P.out_w[0], P.out_w[1],
        st.oz[0], st.os_[0], spec.out_act, tw, pw, P.out_b[0] is not None,
        P.out_b[1] is not None, want_odot=want_odot)
    if want_odot:
        st.odot = odot
    return xbar2, [gW0, gW1], [gb0, gb1]


def reverse2(spec: FusedSpec, P: Params, st: State, tw: Optional[torch.Tensor],
             pw: Optional[torch.Tensor], want_odot: bool = False) -> List[torch.Tensor]:
    """Parameter gradients of sum_n tw_n odot_n + pw_n o_n, in Params.flat()
    order.  tw requires a preceding tangent() and reverse1(seed=tw).
    want_odot makes sure st.odot holds the output tangent afterwards."""
    tangent_on = tw is not None
    graph = st.graph
    dev = st.pos.device
    N = st.pos.shape[0]
    n_lin = len(P.out_w)
    if _out_fused(P):
        xbar2, g_out_w, g_out_b = _out_reverse2(spec, P, st, tw, pw, want_odot)
        return _blocks_reverse2(spec, P, st, tw, xbar2, g_out_w, g_out_b)
    g_out_w = [None] * n_lin
    g_out_b = [None] * n_lin
    # last output linear: o = h W^T (+ b)
    WL = P.out_w[-1]
    gW = torch.zeros_like(WL)
    if tangent_on:
        gW = gW + tw.view(1, -1).mm(st.ohdot[-1])
    if pw is not None:
        gW = gW + pw.view(1, -1).mm(st.oh[-1])
    g_out_w[-1] = gW
    if P.out_b[-1] is not None:
        g_out_b[-1] = (pw.sum().view(1) if pw is not None
                       else torch.zeros_like(P.out_b[-1]))
    hdotbar = tw.view(-1, 1) * WL if tangent_on else None
    hbar2 = pw.view(-1, 1) * WL if pw is not None else torch.zeros(
        N, WL.shape[1], dtype=torch.float32, device=dev)
    for k in range(n_lin - 2, -1, -1):
        d1, d2 = act_derivs(st.oz[k], st.os_[k], spec.out_act)
        zbar2 = hbar2 * d1
        if tangent_on:
            zdotbar = hdotbar * d1
            zbar2 = zbar2 + hdotbar * d2 * st.ozdot[k]
            g_out_w[k] = ops.tmm(zdotbar, st.ohdot[k]) + ops.tmm(zbar2, st.oh[k])
            hdotbar = zdotbar.mm(P.out_w[k])
        else:
            g_out_w[k] = ops.tmm(zbar2, st.oh[k])
        g_out_b[k] = zbar2.sum(0)
        hbar2 = zbar2.mm(P.out_w[k])
    return _blocks_reverse2(spec, P, st, tw, hbar2, g_out_w, g_out_b)


_SIDE_STREAMS = {}
# Weight-gradient reductions of reverse2 on the side stream (False, the
# default, runs them in order on the caller's stream; results are the same bit
# for bit).  Measured on config 2: in order, the eager step's device time is
# 1 % lower (2.351 against 2.376 ms) and the captured step's 0.6 % higher
# (2.353 against 2.338 ms), and no kernel shares the GPU with another stream's
# work while the backward runs, so per-launch times are the kernels' own.
_TMM_SIDE = os.environ.get("MLCG_TMM_SIDE", "0") == "1"


class _SideStream:
    """A second stream (default priority) for the weight-gradient reductions
    of reverse2: their results feed only the optimizer, so they run beside
    the adjoint chain instead of between its kernels.  Each launch waits for
    the work already queued on the main stream; the inputs are held until
    join(), which makes the main stream wait for every side launch, so the
    caching allocator cannot hand their memory to main-stream work the side
    stream has not finished with (this also holds inside a HIP-graph
    capture, where the fork and join become graph edges)."""

    def __init__(self, device: torch.device):
        self.main = torch.cuda.current_stream(device)
        key = (device.index, self.main.cuda_stream)
        if key not in _SIDE_STREAMS:
            _SIDE_STREAMS[key] = torch.cuda.Stream(device=device)
        self.side = _SIDE_STREAMS[key]
        self.held = []

    def run(self, fn, *inputs):
        if not _TMM_SIDE:
            return fn()
        self.side.wait_stream(self.main)
        with torch.cuda.stream(self.side):
            out = fn()
        self.held.extend(t for t in inputs if t is not None)
        return out

    def join(self):
        self.main.wait_stream(self.side)
        self.held.clear()


def _node_tmm_batch(probs, rows, device):
    """The weight-gradient reductions of probs [(a1, b1, a2, b2, colsum)] in
    one batched launch when every operand is a contiguous [rows, 128] fp32
    tensor, else one node_tmm call each (same results up to the split of the
    rows over workgroups)."""
    def ok(t):
        return t is None or (t.dim() == 2 and t.shape[0] == rows
                             and t.shape[1] == ops.NUM_FILTERS and t.dtype == torch.float32
                             and t.is_contiguous())

    if all(ok(t) for pr in probs for t in pr[:4]):
        return ops.node_tmm_batch(probs, rows, device)
    return [ops.node_tmm(a1, b1, a2, b2, colsum=cs) for a1, b1, a2, b2, cs in probs]


def _blocks_reverse2(spec, P, st, tw, xbar2, g_out_w, g_out_b):
    """reverse2 through the interaction blocks from the output network's
    adjoint xbar2; assembles the gradients in Params.flat() order."""
    tangent_on = tw is not None
    graph = st.graph
    n_lin = len(P.out_w)
    g_blocks = [None] * len(P.blocks)
    g_basis = None
    side = _SideStream(st.pos.device)
    N = st.pos.shape[0]

    for k in range(len(P.blocks) - 1, -1, -1):
        bp = P.blocks[k]
        xbar2_in = xbar2
        imgs_t = (_wi(st, k, "A3", True), _wi(st, k, "A2", True))
        if tangent_on:
            zbar2, gagg2 = _lin_dact2_lin(xbar2, bp.A3, st.z[k], st.s[k], spec.block_act,
                                          st.sbar1[k], st.zdot[k], bp.A2, imgs=imgs_t)
        else:
            zbar2, gagg2 = _lin_dact2_lin(xbar2, bp.A3, st.z[k], st.s[k], spec.block_act,
                                          None, None, bp.A2, imgs=imgs_t)
        g1 = st.gagg1[k] if tangent_on else None
        yd = st.ydot[k] if tangent_on else None
        dd = st.ddot if tangent_on else None
        ybar2, _, _ = ops.cfconv_gather_rev2(gagg2, g1, st.y[k], yd, st.W[k], st.Wd[k], dd,
                                             graph, pair_adjoints=False)
        # the block's three weight-gradient reductions (lin, conv.lin2 with
        # their biases, conv.lin1), one batched launch on the side stream
        if tangent_on:
            probs = [(xbar2_in, st.s[k], st.xbar_out[k], st.sdot[k], True),
                     (zbar2, st.agg[k], st.zbar1[k], st.aggdot[k], True),
                     (ybar2, st.x[k], st.ybar1[k], st.xdot_in[k], False)
                     if st.xdot_in[k] is not None else (ybar2, st.x[k], None, None, False)]
        else:
            probs = [(xbar2_in, st.s[k], None, None, True), (zbar2, st.agg[k], None, None, True),
                     (ybar2, st.x[k], None, None, False)]
        held = [t for pr in probs for t in pr[:4]]
        (gA3, gc3), (gA2, gc2), gA1 = side.run(
            lambda: _node_tmm_batch(probs, N, st.pos.device), *held)
        xbar2 = ops.node_linear(ybar2, bp.A1, transpose=True, residual=xbar2,
                                w_image=_wi(st, k, "A1", True))
        res = ops.filter_bwd_cfconv(st.pos, graph, st.filt, bp.W1, bp.b1, bp.W2, gagg2,
                                    st.y[k], g1, yd, dd, pair_adjoints=spec.basis_trainable,
                                    strict_fp32=spec.strict_fp32)
        gW1, gb1, gW2 = res[:3]
        if spec.basis_trainable:
            # basis parameters are shared by all blocks: accumulate
            g_basis = ops.rbf_param_grad(st.dist, graph, st.filt, bp.W1, res[3], res[4],
                                         out=g_basis)
        g_blocks[k] = [gW1, gb1, gW2, gA1, gA2, gc2, gA3, gc3]
    if P.emb.shape[0] <= 128 and P.emb.shape[1] == 128 and st.types.dtype == torch.int64:
        # fixed summation order; an out-of-table type raises a numerics flag
        g_emb = ops.type_sum(xbar2, st.types, P.emb.shape[0], want_bad=False)[0]
    else:
        g_emb = torch.zeros_like(P.emb).index_add_(0, st.types, xbar2)
    side.join()
    out = [g_emb]
    for gb in g_blocks:
        out += gb
    for k in range(n_lin):
        out.append(g_out_w[k])
        if P.out_b[k] is not None:
            out.append(g_out_b[k])
    if spec.basis_trainable:
        gc, gw = g_basis
        if P.basis[1].numel() != gw.numel():  # one shared Gaussian coefficient
            gw = gw.sum()
        out += [gc.reshape(P.basis[0].shape).to(P.basis[0].dtype),
                gw.reshape(P.basis[1].shape).to(P.basis[1].dtype)]
    return out


_ONES: dict = {}


def _ones(n: int, device: torch.device) -> torch.Tensor:
    """A read-only float32 vector of n ones on device, made once per stream
    (outside any stream capture, and filled on the stream that first uses it)
    and then shared: the unit node seeds of the force path."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, n, torch.cuda.current_stream(device).cuda_stream)
    t = _ONES.get(key)
    if t is None:
        t = torch.ones(n, dtype=torch.float32, device=device)
        if not torch.cuda.is_current_stream_capturing():
            # one made inside a capture holds its ones only once the graph
            # has been replayed, so it is not kept for eager callers
            _ONES[key] = t
    return t


def node_seed(frame_weights: torch.Tensor, batch: torch.Tensor) -> torch.Tensor:
    return frame_weights.to(torch.float32).index_select(0, batch).contiguous()


# --------------------------------------------------------------------------
# autograd glue

class EnergyForces(torch.autograd.Function):
    """(E [B], F [N, 3]) = fused SchNet energies and forces.

    backward(Ebar, Fbar) returns parameter gradients of
    <Ebar, E> + <Fbar, F>, i.e. the force-matching double backward.  Position
    gradients are not produced (positions enter detached)."""

    @staticmethod
    def forward(ctx, spec, pos, types, batch, graph, training, *flat):
        P = Params.unflat(spec, list(flat))
        ones = _ones(pos.shape[0], pos.device)
        E, st = forward(spec, P, pos, types, graph, save=True, rev_seed=ones)
        F = reverse1(spec, P, st, ones, keep_adjoints=bool(training))
        if training:
            ctx.spec, ctx.P, ctx.st, ctx.batch = spec, P, st, batch
        ctx.set_materialize_grads(False)
        return E, F

    @staticmethod
    def backward(ctx, Ebar, Fbar):
        spec, P, st, batch = ctx.spec, ctx.P, ctx.st, ctx.batch
        if spec.f16:
            raise NotImplementedError(
                "the fp16 filter path provides energies and forces only; "
                "train with fp32 filters")
        tw = pw = None
        if Fbar is not None:
            # <Fbar, F> = <Fbar, -grad sum E> : tangent along u = -Fbar, seed 1
            tangent(spec, P, st, Fbar, scale=-1.0)
            tw = _ones(st.pos.shape[0], st.pos.device)
        if Ebar is not None:
            pw = node_seed(Ebar, batch)
        if tw is None and pw is None:
            grads = [None] * len(P.flat())
        else:
            grads = reverse2(spec, P, st, tw, pw)
        ctx.st = None
        return (None, None, None, None, None, None, *grads)


class Energy(torch.autograd.Function):
    """E [B] with a first-order backward that is itself differentiable
    (EnergyGrad), for generic autograd.grad(E, pos, create_graph=True) use."""

    @staticmethod
    def forward(ctx, spec, types, batch, graph, pos, *flat):
        P = Params.unflat(spec, list(flat))
        E, st = forward(spec, P, pos.detach(), types, graph, save=True)
        ctx.spec, ctx.P, ctx.st, ctx.batch = spec, P, st, batch
        ctx.save_for_backward(pos, *flat)
        return E

    @staticmethod
    def backward(ctx, Ebar):
        pos, *flat = ctx.saved_tensors
        out = EnergyGrad.apply(ctx.spec, ctx.st, ctx.batch, Ebar, pos, *flat)
        return (None, None, None, None, *out)


class EnergyGrad(torch.autograd.Function):
    """(dE/dpos, dE/dtheta) weighted by Ebar; its backward implements the
    second-order term for a loss on dE/dpos (tangent + reverse2)."""

    @staticmethod
    def forward(ctx, spec, st, batch, Ebar, pos, *flat):
        P = Params.unflat(spec, list(flat))
        seed = node_seed(Ebar, batch)
        F = reverse1(spec, P, st, seed)
        pgrads = reverse2(spec, P, st, None, seed)
        ctx.spec, ctx.st, ctx.P, ctx.seed, ctx.batch = spec, st, P, seed, batch
        ctx.set_materialize_grads(False)
        return (-F, *pgrads)

    @staticmethod
    def backward(ctx, gpos_bar, *pgrad_bars):
        if any(g is not None for g in pgrad_bars):
            raise NotImplementedError(
                "differentiating parameter gradients of the fused SchNet is not supported")
        spec, st, P = ctx.spec, ctx.st, ctx.P
        nflat = len(P.flat())
        if gpos_bar is None:
            return (None,) * (5 + nflat)
        if spec.f16:
            raise NotImplementedError("the fp16 filter path has no double backward")
        # d/dtheta <gpos_bar, grad_pos(sum seed o)> = tangent along gpos_bar
        tangent(spec, P, st, gpos_bar)
        grads = reverse2(spec, P, st, ctx.seed, None, want_odot=True)
        # d/dEbar_b <gpos_bar, grad E_b> = per-frame tangent of the energy
        Ebar_grad = ops.segment_sum(st.odot, st.graph.frame_ptr)
        return (None, None, None, Ebar_grad, None, *grads)
