"""Host-side wrappers around the C ABI of ``libmlcg_hip.so``.

Every function validates shapes, dtypes, devices and contiguity (raising
``RuntimeError`` like the reference's ``AT_ASSERTM`` checks,
``src/opt_radius/mlcg_opt_radius/radius.cu:205-228``), allocates outputs with
torch's caching allocator and launches on torch's current stream.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch

from . import _lib
from ._lib import call, ptr, require_device, stream_handle

NUM_FILTERS = 128  # F fixed by the MFMA tiling of the filter kernels


def _check(cond: bool, msg) -> None:
    """Raise RuntimeError(msg) unless cond; msg may be a zero-argument
    callable, so that a message needing formatting costs nothing when the
    check passes."""
    if not cond:
        raise RuntimeError(msg() if callable(msg) else msg)


def _as_i64(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.int64).contiguous()


@dataclass
class PairGraph:
    """Canonical radius graph plus the receiver CSR and pair map.

    edge_index : [2, E] int64, rows (centre i, neighbour j), sorted by (i, j)
    rowptr     : [N + 1] int32, CSR offsets of rows of edge_index
    col        : [E] int32 = edge_index[1]
    pair_ij    : [2, P] int32, the upper edges (i < j) in canonical order
    pairptr    : [N + 1] int32, offsets of each node's upper edges in pair_ij
    eid2pair   : [E] int32, pair id of every directed edge
    frame_ptr  : [B + 1] int64
    """

    edge_index: torch.Tensor
    rowptr: torch.Tensor
    col: Optional[torch.Tensor]
    pair_ij: Optional[torch.Tensor]
    pairptr: Optional[torch.Tensor]
    eid2pair: Optional[torch.Tensor]
    frame_ptr: torch.Tensor
    num_nodes: int
    num_edges: int
    num_pairs: int
    overflow: int = 0
    flags: Optional[torch.Tensor] = None  # device int32 [1]: overflow bits

    @property
    def n_pairs_dev(self) -> torch.Tensor:
        """One-element int32 view holding the live pair count on the device."""
        return self.pairptr[self.num_nodes:]

    @property
    def pair_capacity(self) -> int:
        return 0 if self.pair_ij is None else self.pair_ij.shape[1]


def frame_ptr_from_batch(batch: torch.Tensor, n_frames: int) -> torch.Tensor:
    """frame_ptr [B+1] from a sorted batch vector (radius.py:72-75 equivalent)."""
    require_device(batch)
    batch = _as_i64(batch)
    out = torch.empty(n_frames + 1, dtype=torch.int64, device=batch.device)
    call("mlcg_frame_ptr_from_batch", ptr(batch), batch.numel(), n_frames, ptr(out),
         stream_handle(batch.device))
    return out


def exclusion_pair_to_ptr(exc_pair_index: torch.Tensor,
                          num_nodes: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(pair_xs [M] int64, y_ptr [num_nodes + 1] int64): the per-centre CSR of
    an exclusion pair list [2, M] (row 0 = excluded neighbour x, row 1 =
    centre y), ordered by y then x, on the input's device.

    Same contract as the reference's ``mlcg::exclusion_pair_to_ptr``
    (exclusion_pairs.cpp:7-62): int64 input of shape [2, M], conversion on
    the host, a RuntimeError for a negative centre index."""
    _check(exc_pair_index.dtype == torch.int64, "exc_pair_index must be int64")
    _check(exc_pair_index.dim() == 2 and exc_pair_index.shape[0] == 2,
           f"exc_pair_index must be [2, M], got {tuple(exc_pair_index.shape)}")
    _check(num_nodes >= 0, "num_nodes must be non-negative")
    host = exc_pair_index.detach().cpu().contiguous()
    m = host.shape[1]
    pair_xs = torch.empty(m, dtype=torch.int64)
    y_ptr = torch.empty(num_nodes + 1, dtype=torch.int64)
    call("mlcg_exclusion_pair_to_ptr", ptr(host) if m else None, m, int(num_nodes),
         ptr(pair_xs) if m else None, ptr(y_ptr))
    dev = exc_pair_index.device
    return pair_xs.to(dev), y_ptr.to(dev)


def _validate_exclusions(exclude_pair_xs, ptr_exclude_pair_xs, n: int, dev):
    if exclude_pair_xs is None and ptr_exclude_pair_xs is None:
        return None, None
    _check(exclude_pair_xs is not None and ptr_exclude_pair_xs is not None,
           "exclude_pair_xs and ptr_exclude_pair_xs go together")
    for t, name in ((exclude_pair_xs, "exclude_pair_xs"),
                    (ptr_exclude_pair_xs, "ptr_exclude_pair_xs")):
        require_device(t)
        _check(t.device == dev, f"{name} must be on {dev}")
        _check(t.dtype == torch.int64 and t.dim() == 1, f"{name} must be 1-D int64")
    _check(ptr_exclude_pair_xs.numel() == n + 1,
           f"ptr_exclude_pair_xs must have N + 1 = {n + 1} entries")
    xs = exclude_pair_xs.contiguous()
    eptr = ptr_exclude_pair_xs.contiguous()
    if not torch.cuda.is_current_stream_capturing():
        # the kernels read xs[eptr[i] .. eptr[i+1]) unchecked: make sure every
        # segment lies inside xs (one host synchronisation, outside capture)
        ok = torch.stack([(eptr[1:] >= eptr[:-1]).all(), eptr[0] >= 0,
                          eptr[-1] <= xs.numel()]).all()
        _check(bool(ok), "ptr_exclude_pair_xs must be non-decreasing, start at >= 0 and end "
               "at <= len(exclude_pair_xs)")
    if xs.numel() == 0:  # keep a valid address for the kernels
        xs = torch.zeros(1, dtype=torch.int64, device=dev)
    return xs, eptr


def _validate_pos(pos: torch.Tensor) -> torch.Tensor:
    require_device(pos)
    _check(pos.dim() == 2 and pos.shape[1] == 3, lambda: f"pos must be [N, 3], got {tuple(pos.shape)}")
    _check(pos.dtype == torch.float32,
           f"the HIP radius graph and CFConv kernels take float32 positions, got {pos.dtype}")
    return pos.contiguous()


def radius_flags_read(overflow: int) -> None:
    """Host-side bookkeeping for radius-graph flags read back from the device:
    after bit 8 (a look-back wait hit its bound) the cached look-back
    workspaces are discarded -- a block that had not started when the last
    block advanced the workspace header may have published into the next
    launch's status array -- so the next call starts from a zero-filled one.
    Every caller that reads the flags calls this before raising."""
    if overflow & 8:
        _RADIUS_WS.clear()


def radius_flags_message(overflow: int, capacity=None) -> str:
    """What the radius-graph flag bits of `overflow` mean."""
    parts = []
    if overflow & 1:
        parts.append("a row reached max_num_neighbors")
    if overflow & 2:
        parts.append("more edges than the capacity" +
                     (f" {capacity}" if capacity is not None else ""))
    if overflow & 4:
        parts.append("the exclusion list is not symmetric")
    if overflow & 8:
        parts.append("a look-back wait of the radius kernel hit its bound")
    if overflow & 16:
        parts.append("more than 2^31 - 1 edges for the int32 CSR")
    return "; ".join(parts) if parts else "none"


def _check_radius_flags(overflow: int) -> None:
    """Raise for the radius graph's internal failure bits (8: a look-back wait
    hit its bound, 16: more than 2^31 - 1 edges for the int32 CSR)."""
    if overflow & 16:
        raise RuntimeError("radius graph: more than 2^31 - 1 edges; the int32 CSR cannot "
                           "hold them")
    if overflow & 8:
        raise RuntimeError("radius graph: a block of the sizing pass timed out waiting for "
                           "its predecessors")


# Look-back workspaces of the radius graph, one per (device, stream): zero-filled
# once, and every call leaves its workspace ready for the next call on that
# stream (mlcg_radius_workspace_bytes).
_RADIUS_WS: dict = {}


# Workspaces zero-filled ahead of a stream capture (reserve_radius_workspaces),
# per device, handed to the radius-graph calls made inside it.
_CAPTURE_WS: dict = {}


def reserve_radius_workspaces(n: int, dev: torch.device, count: int) -> List[torch.Tensor]:
    """Zero-filled look-back workspaces for `count` radius-graph calls over n
    rows made inside the stream capture that follows on dev: those calls take
    them (in order) instead of recording a zero fill that every replay of the
    graph would run.  The caller keeps the list alive as long as the graph,
    zeroes them again after a look-back timeout (flag 8), and ends the
    reservation with release_radius_workspaces(dev) after the capture."""
    words = max(1, _lib.load().mlcg_radius_workspace_bytes(n) // 8)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = [torch.zeros(words, dtype=torch.int64, device=dev) for _ in range(count)]
    _CAPTURE_WS[index] = list(ws)
    return ws


def release_radius_workspaces(dev: torch.device) -> None:
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    _CAPTURE_WS.pop(index, None)


def _radius_workspace(n: int, dev: torch.device) -> Tuple[torch.Tensor, Optional[tuple]]:
    """The workspace for n rows on the current stream, and its cache key
    (None for a fresh one).  Inside a stream capture the graph gets a
    workspace of its own (its replays may run on any stream): a reserved one
    (reserve_radius_workspaces) or a zero-filled one."""
    words = max(1, _lib.load().mlcg_radius_workspace_bytes(n) // 8)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    if torch.cuda.is_current_stream_capturing():
        pool = _CAPTURE_WS.get(index, [])
        for i, ws in enumerate(pool):
            if ws.numel() >= words:
                return pool.pop(i), None
        return torch.zeros(words, dtype=torch.int64, device=dev), None
    key = (index, torch.cuda.current_stream(dev).cuda_stream)
    ws = _RADIUS_WS.get(key)
    if ws is None or ws.numel() < words:
        ws = torch.zeros(words, dtype=torch.int64, device=dev)
        _RADIUS_WS[key] = ws
    return ws, key


def radius_graph(
    pos: torch.Tensor,
    r: float,
    batch: Optional[torch.Tensor] = None,
    loop: bool = False,
    max_num_neighbors: int = 32,
    with_pairs: bool = False,
    n_frames: Optional[int] = None,
    frame_ptr: Optional[torch.Tensor] = None,
    capacity: Optional[int] = None,
    exclude_pair_xs: Optional[torch.Tensor] = None,
    ptr_exclude_pair_xs: Optional[torch.Tensor] = None,
) -> PairGraph:
    """All pairs (i, j) of the same frame with |pos[j] - pos[i]| < r.

    Drop-in for ``torch_cluster.radius_graph(pos, r, batch, loop,
    max_num_neighbors, flow="target_to_source")`` as called at
    ``mlcg/neighbor_list/torch_impl.py:216-224``, with a deterministic
    canonical order (i ascending, then j ascending).  The membership test is
    ``d2 < fl32(r*r)`` with d2 = ((dx*dx + dy*dy) + dz*dz) in fp32, or in fp64
    (``d2 < r*r``) for float64 positions, or for float16 / bfloat16 positions
    with every operation rounded to the 16-bit type as the reference's
    Half / BFloat16 kernels compute it (edge list only, no pair structures;
    the 16-bit forms size their output exactly, without ``capacity``).

    with_pairs additionally builds the receiver CSR and pair map used by the
    CFConv kernels (it requires a symmetric graph, i.e. no binding
    ``max_num_neighbors`` and ``loop=False``).

    Without ``capacity`` the edge count is read back to size the outputs
    exactly (one host synchronisation, as the reference's radius.cu:288).
    With ``capacity`` nothing synchronises: buffers hold ``capacity`` edges
    (``capacity // 2`` pairs), the live counts stay on the device
    (``rowptr[N]``, ``n_pairs_dev``), rows are clamped to the capacity so
    every later kernel stays in bounds, and ``graph.flags`` (bit 0: a row
    exceeded max_num_neighbors, bit 1: the capacity was exceeded) must be
    checked by the caller -- this is the form a captured graph replays.

    ``exclude_pair_xs`` / ``ptr_exclude_pair_xs`` (int64, the CSR of
    ``exclusion_pair_to_ptr``) drop listed neighbours from each row as the
    reference's native kernel does (radius.cu:113-133); excluded neighbours
    do not count towards ``max_num_neighbors``.  With ``with_pairs`` the
    exclusions must be symmetric (flag bit 2 otherwise).
    """
    f64 = pos.dtype == torch.float64
    narrow = pos.dtype in (torch.float16, torch.bfloat16)
    sfx = {torch.float64: "_f64", torch.float16: "_f16", torch.bfloat16: "_bf16"}.get(
        pos.dtype, "")
    if f64 or narrow:
        # the membership test in the positions' own arithmetic (the reference
        # dispatches on the scalar type, radius.cu:243-250); edge list only
        require_device(pos)
        _check(pos.dim() == 2 and pos.shape[1] == 3,
               f"pos must be [N, 3], got {tuple(pos.shape)}")
        _check(not with_pairs, "the CFConv pair structures take float32 positions")
        _check(not (narrow and capacity is not None),
               "the fixed-capacity radius graph takes float32 or float64 positions")
        pos = pos.contiguous()
    else:
        pos = _validate_pos(pos)
    n = pos.shape[0]
    dev = pos.device
    if batch is None:
        batch = torch.zeros(n, dtype=torch.int64, device=dev)
    require_device(batch)
    _check(batch.dim() == 1 and batch.numel() == n, "batch must be [N]")
    batch = _as_i64(batch)
    _check(r >= 0, "r must be non-negative")
    _check(max_num_neighbors >= 0, "max_num_neighbors must be non-negative")
    if with_pairs:
        _check(not loop, "the pair map is defined for graphs without self loops")
    if capacity is not None:
        _check(capacity >= 0 and capacity < 2 ** 31, "capacity must fit int32 edge ids")
    if frame_ptr is None:
        if n_frames is None:
            n_frames = int(batch[-1].item()) + 1 if n > 0 else 0
        frame_ptr = frame_ptr_from_batch(batch, n_frames)
    exs, eptr = _validate_exclusions(exclude_pair_xs, ptr_exclude_pair_xs, n, dev)
    s = stream_handle(dev)

    mnn = int(max_num_neighbors)
    rowptr = torch.empty(n + 1, dtype=torch.int32, device=dev)
    pairptr = torch.empty(n + 1, dtype=torch.int32, device=dev) if with_pairs else None
    flags = torch.empty(1, dtype=torch.int32, device=dev)  # cleared by the kernels
    ws, ws_key = _radius_workspace(n, dev)
    if capacity is None:
        # sizing pass (counts, block scan, look-back) -> rowptr / pairptr, then
        # one host sync to size the outputs (the reference syncs at radius.cu:288)
        if narrow:
            call(f"mlcg_radius_rowptr{sfx}", ptr(pos), ptr(batch), ptr(frame_ptr), n, float(r),
                 int(loop), mnn, ptr(exs), ptr(eptr), ptr(rowptr), ptr(ws), ptr(flags), s)
        else:
            call(f"mlcg_radius_rowptr{sfx}", ptr(pos), ptr(batch), ptr(frame_ptr), n, float(r),
                 int(loop), mnn, ptr(exs), ptr(eptr), ptr(rowptr), ptr(pairptr), ptr(ws),
                 ptr(flags), s)
        if with_pairs:
            e_count, p_count, overflow = torch.cat([rowptr[n:], pairptr[n:], flags]).tolist()
        else:
            (e_count, overflow), p_count = torch.cat([rowptr[n:], flags]).tolist(), 0
        radius_flags_read(overflow)
        _check_radius_flags(overflow)
        if with_pairs and overflow & 1:
            raise RuntimeError(
                f"max_num_neighbors={max_num_neighbors} binds: the truncated graph is not "
                "symmetric and the pair-based CFConv kernels cannot use it; raise "
                "max_num_neighbors")
        if with_pairs and overflow & 4:
            raise RuntimeError(
                "the exclusion list is not symmetric: an edge (i, j) is kept while (j, i) is "
                "excluded, and the pair-based CFConv kernels need a symmetric graph")
        e_cap, p_cap = e_count, p_count
    else:
        e_cap, p_cap = capacity, capacity // 2
        e_count = p_count = -1  # live counts stay on the device
        overflow = -1
    edge_index = torch.empty(2, e_cap, dtype=torch.int64, device=dev)
    col = pair_ij = eid2pair = None
    if with_pairs:
        col = torch.empty(e_cap, dtype=torch.int32, device=dev)
        pair_ij = torch.empty(2, p_cap, dtype=torch.int32, device=dev)
        eid2pair = torch.empty(e_cap, dtype=torch.int32, device=dev)
    if capacity is None:
        if f64 or narrow:
            call(f"mlcg_radius_fill{sfx}", ptr(pos), ptr(batch), ptr(frame_ptr), n, float(r),
                 int(loop), mnn, ptr(exs), ptr(eptr), ptr(rowptr), e_cap, e_cap,
                 ptr(edge_index), ptr(flags), s)
        else:
            call("mlcg_radius_fill", ptr(pos), ptr(batch), ptr(frame_ptr), n, float(r),
                 int(loop), mnn, ptr(exs), ptr(eptr), ptr(rowptr), ptr(pairptr), e_cap, e_cap,
                 ptr(edge_index), ptr(col), p_cap, p_cap, ptr(pair_ij), ptr(eid2pair),
                 ptr(flags), s)
    elif f64:
        # one launch: sweep, look-back and write; the CSR comes out clamped to
        # the capacity, so every consumer stays inside the buffers
        call("mlcg_radius_graph_f64", ptr(pos), ptr(batch), ptr(frame_ptr), n, float(r),
             int(loop), mnn, ptr(exs), ptr(eptr), ptr(rowptr), e_cap, e_cap, ptr(edge_index),
             ptr(ws), ptr(flags), s)
    else:
        call("mlcg_radius_graph", ptr(pos), ptr(batch), ptr(frame_ptr), n, float(r), int(loop),
             mnn, ptr(exs), ptr(eptr), ptr(rowptr), ptr(pairptr), e_cap, e_cap,
             ptr(edge_index), ptr(col), p_cap, p_cap, ptr(pair_ij), ptr(eid2pair), ptr(ws),
             ptr(flags), s)
    if with_pairs:
        call("mlcg_pair_reverse_map", ptr(pair_ij), p_cap, ptr(pairptr[n:]), p_cap,
             ptr(rowptr), ptr(col), ptr(eid2pair), s)
    return PairGraph(edge_index=edge_index, rowptr=rowptr, col=col, pair_ij=pair_ij,
                     pairptr=pairptr, eid2pair=eid2pair,
                     frame_ptr=frame_ptr, num_nodes=n, num_edges=e_count,
                     num_pairs=p_count if with_pairs else 0, overflow=int(overflow),
                     flags=flags)


# --------------------------------------------------------------------------
# Reductions over long row dimensions

SPLIT_ROWS = 4096  # rows per slice of the split-K products below


def tmm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a^T b for a [R, M], b [R, N] with R >> M, N (weight gradients summed
    over pairs or nodes).  The row dimension is cut into fixed slices whose
    products run as one batched GEMM and are then summed in slice order, so
    the result is deterministic and the library GEMM sees a well-shaped
    problem instead of a single M x N tile with an enormous K."""
    R = a.shape[0]
    S = R // SPLIT_ROWS
    if S < 2:
        return a.t().mm(b)
    m = S * SPLIT_ROWS
    av = a[:m].reshape(S, SPLIT_ROWS, a.shape[1])
    bv = b[:m].reshape(S, SPLIT_ROWS, b.shape[1])
    out = torch.bmm(av.transpose(1, 2), bv).sum(0)
    if m < R:
        out = out + a[m:].t().mm(b[m:])
    return out


# --------------------------------------------------------------------------
# Node-level linears (products on hipBLASLt, weight gradients on the MFMA
# reduction kernel for F = 128)

def node_linear(x: torch.Tensor, W: torch.Tensor, bias: Optional[torch.Tensor] = None,
                residual: Optional[torch.Tensor] = None, transpose: bool = False,
                w_image: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x W^T (or x W with transpose=True) [+ bias] [+ residual]: the fused
    node GEMM kernel for [N, 128] x [128, 128] (w_image: W's split image for
    this orientation, node_weight_images); other shapes (the output network)
    go to one library GEMM with the epilogue terms in addmm's beta input."""
    require_device(x)
    if _node_gemm_ok(x, W):
        return node_gemm(x, W, transpose=transpose, bias=bias, residual=residual,
                         w_image=w_image)[0]
    Wm = W if transpose else W.t()
    if residual is not None and bias is not None:
        return torch.addmm(residual + bias, x, Wm)
    if residual is not None:
        return torch.addmm(residual, x, Wm)
    if bias is not None:
        return torch.addmm(bias, x, Wm)
    return x.mm(Wm)


NODE_PLAIN, NODE_ACT, NODE_DACT, NODE_DACT2 = 0, 1, 2, 3


def _node_gemm_ok(x: torch.Tensor, W: torch.Tensor) -> bool:
    return (x.is_cuda and x.dtype == torch.float32 and x.dim() == 2
            and x.shape[1] == NUM_FILTERS and tuple(W.shape) == (NUM_FILTERS, NUM_FILTERS))


def node_gemm(x: torch.Tensor, W: torch.Tensor, transpose: bool = False,
              bias: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
              epilogue: int = NODE_PLAIN, act: int = 0, z: Optional[torch.Tensor] = None,
              s: Optional[torch.Tensor] = None, e: Optional[torch.Tensor] = None,
              f: Optional[torch.Tensor] = None, want_out0: bool = True,
              w_image: Optional[torch.Tensor] = None,
              ) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
    """(out0, out1) of the fused node GEMM (mlcg_node_gemm) on [N, 128] fp32
    rows and a [128, 128] weight: y = x W^T (x W with transpose) [+ bias]
    [+ residual], then the epilogue

        NODE_PLAIN  out0 = y
        NODE_ACT    out0 = y, out1 = act(y)
        NODE_DACT   out0 = y, out1 = y * act'(z)
        NODE_DACT2  out0 = y * act'(z) [+ e * act''(z) * f]

    (act' and act'' from z and s = act(z)).  out0 is skipped for ACT/DACT
    when want_out0 is False.  w_image: W's split image for this orientation
    (node_weight_images, made after W's last change), read instead of
    splitting W in the kernel; the results are the same bit for bit."""
    require_device(x)
    _check(_node_gemm_ok(x, W), lambda: f"node_gemm takes [N, {NUM_FILTERS}] float32 rows and a "
           f"[{NUM_FILTERS}, {NUM_FILTERS}] weight, got {tuple(x.shape)} / {tuple(W.shape)}")
    n = x.shape[0]
    dev = x.device
    c = lambda t: None if t is None else t.contiguous()  # noqa: E731
    x, W, bias, residual, z, s, e, f = map(c, (x, W, bias, residual, z, s, e, f))
    for t in (residual, z, s, e, f):
        _check(t is None or (t.shape == x.shape and t.dtype == torch.float32
                             and t.device == dev), "epilogue tensors must match x")
    _check(bias is None or bias.numel() == NUM_FILTERS, "bias must have 128 entries")
    out0 = out1 = None
    if epilogue == NODE_PLAIN or epilogue == NODE_DACT2 or want_out0:
        out0 = torch.empty_like(x)
    if epilogue in (NODE_ACT, NODE_DACT):
        out1 = torch.empty_like(x)
    _check_w_image(w_image, dev)
    call("mlcg_node_gemm", ptr(x), n, NUM_FILTERS, ptr(W), int(transpose), ptr(bias),
         ptr(residual), int(epilogue), int(act), ptr(z), ptr(s), ptr(e), ptr(f), ptr(out0),
         ptr(out1), ptr(w_image), stream_handle(dev),
         work=_node_gemm_bytes(n, epilogue, act, (x, residual, out0, out1), s, z, e, f, 1))
    return out0, out1


def _node_gemm_bytes(n, epilogue, act, tensors, s, z, e, f, n_weights):
    """Algorithmic HBM bytes of one node-GEMM launch: every [n, 128] fp32
    tensor the launch reads or writes once (the epilogue's z only for
    activations other than tanh, whose derivatives come from s alone), the
    weights and biases once."""
    rows = [t for t in tensors if t is not None]
    if epilogue in (NODE_DACT, NODE_DACT2):
        rows += [t for t in (s, None if act == 0 else z) if t is not None]
        if epilogue == NODE_DACT2:
            rows += [t for t in (e, f) if t is not None]
    return 4 * NUM_FILTERS * n * len(rows) + n_weights * 4 * (NUM_FILTERS + 1) * NUM_FILTERS


def node_gemm2(x: torch.Tensor, W: torch.Tensor, W2: torch.Tensor, transpose: bool = False,
               bias: Optional[torch.Tensor] = None, residual: Optional[torch.Tensor] = None,
               epilogue: int = NODE_ACT, act: int = 0, z: Optional[torch.Tensor] = None,
               s: Optional[torch.Tensor] = None, e: Optional[torch.Tensor] = None,
               f: Optional[torch.Tensor] = None, want_out0: bool = True,
               bias2: Optional[torch.Tensor] = None, residual2: Optional[torch.Tensor] = None,
               w_image: Optional[torch.Tensor] = None, w2_image: Optional[torch.Tensor] = None,
               want_out1: bool = True,
               ) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor], torch.Tensor]:
    """(out0, out1, out2): node_gemm(x, W, ...) with an ACT, DACT or DACT2
    epilogue followed, in the same kernel (mlcg_node_gemm2), by
    out2 = v W2^T (v W2 with transpose) [+ bias2] [+ residual2], v being out1
    (ACT, DACT) or out0 (DACT2).  Bit-identical to the two node_gemm calls.
    w_image, w2_image: split images of W and W2 as in node_gemm.  With the
    DACT epilogue, want_out1=False leaves v (out1) unwritten (None)."""
    require_device(x)
    _check(epilogue in (NODE_ACT, NODE_DACT, NODE_DACT2),
           "node_gemm2 takes an ACT, DACT or DACT2 first epilogue")
    _check(_node_gemm_ok(x, W) and _node_gemm_ok(x, W2),
           lambda: f"node_gemm2 takes [N, {NUM_FILTERS}] float32 rows and two "
           f"[{NUM_FILTERS}, {NUM_FILTERS}] weights, got {tuple(x.shape)} / "
           f"{tuple(W.shape)} / {tuple(W2.shape)}")
    n = x.shape[0]
    dev = x.device
    c = lambda t: None if t is None else t.contiguous()  # noqa: E731
    x, W, W2, bias, bias2, residual, residual2, z, s, e, f = map(
        c, (x, W, W2, bias, bias2, residual, residual2, z, s, e, f))
    for t in (residual, residual2, z, s, e, f):
        _check(t is None or (t.shape == x.shape and t.dtype == torch.float32
                             and t.device == dev), "epilogue tensors must match x")
    for b in (bias, bias2):
        _check(b is None or b.numel() == NUM_FILTERS, "bias must have 128 entries")
    out0 = out1 = None
    if epilogue == NODE_DACT2 or want_out0:
        out0 = torch.empty_like(x)
    if epilogue == NODE_ACT or (epilogue == NODE_DACT and want_out1):
        out1 = torch.empty_like(x)
    out2 = torch.empty_like(x)
    _check_w_image(w_image, dev)
    _check_w_image(w2_image, dev)
    call("mlcg_node_gemm2", ptr(x), n, NUM_FILTERS, ptr(W), int(transpose), ptr(bias),
         ptr(residual), int(epilogue), int(act), ptr(z), ptr(s), ptr(e), ptr(f), ptr(out0),
         ptr(out1), ptr(W2), ptr(bias2), ptr(residual2), ptr(out2), ptr(w_image),
         ptr(w2_image), stream_handle(dev),
         work=_node_gemm_bytes(n, epilogue, act, (x, residual, out0, out1, residual2, out2),
                               s, z, e, f, 2))
    return out0, out1, out2


NODE_W_IMAGE_HALFS = 32768  # fp16 entries of one split weight image (64 KiB)


def _check_w_image(img: Optional[torch.Tensor], dev) -> None:
    _check(img is None or (img.dtype == torch.float16 and img.device == dev
                           and img.numel() == NODE_W_IMAGE_HALFS and img.is_contiguous()
                           and img.data_ptr() % 16 == 0),
           lambda: f"a node weight image is a contiguous [{NODE_W_IMAGE_HALFS}] float16 tensor "
                   f"on {dev} (node_weight_images)")


def node_weight_images(weights, transposes) -> torch.Tensor:
    """[count, NODE_W_IMAGE_HALFS] fp16: the split operand image of each
    [128, 128] fp32 weight for node_gemm / node_gemm2 in the orientation given
    by its transpose flag, all made in one launch (mlcg_node_weight_images,
    at most 32 per launch).  Row k is the w_image argument for weights[k]."""
    _check(len(weights) == len(transposes), "one transpose flag per weight")
    n = len(weights)
    _check(n >= 1, "node_weight_images needs at least one weight")
    dev = weights[0].device
    ws = []
    for W in weights:
        _check(W.is_cuda and W.device == dev and W.dtype == torch.float32
               and tuple(W.shape) == (NUM_FILTERS, NUM_FILTERS),
               lambda: f"node weights must be [{NUM_FILTERS}, {NUM_FILTERS}] float32 on {dev}")
        ws.append(W.detach().contiguous())
    out = torch.empty(n, NODE_W_IMAGE_HALFS, dtype=torch.float16, device=dev)
    for k in range(0, n, 32):
        m = min(32, n - k)
        warr = (ctypes.c_void_p * m)(*[t.data_ptr() for t in ws[k:k + m]])
        tarr = (ctypes.c_int * m)(*[int(bool(t)) for t in transposes[k:k + m]])
        call("mlcg_node_weight_images", warr, tarr, m, ptr(out[k]), stream_handle(dev))
    return out


def node_tmm(a1: torch.Tensor, b1: torch.Tensor, a2: Optional[torch.Tensor] = None,
             b2: Optional[torch.Tensor] = None, colsum: bool = False):
    """a1^T b1 (+ a2^T b2) reduced over the rows; with colsum, returns
    (product, a1.sum(0)) from the same pass."""
    require_device(a1, b1, a2, b2)
    shapes_ok = all(t is None or (t.dim() == 2 and t.shape[1] == NUM_FILTERS)
                    for t in (a1, b1, a2, b2))
    if shapes_ok and a1.is_cuda and a1.dtype == torch.float32:
        rows = a1.shape[0]
        out = torch.empty(NUM_FILTERS, NUM_FILTERS, dtype=torch.float32, device=a1.device)
        cs = torch.empty(NUM_FILTERS, dtype=torch.float32, device=a1.device) if colsum else None
        nws = int(_lib.load().mlcg_node_tmm_workspace_floats(rows))
        ws = torch.empty(nws, dtype=torch.float32, device=a1.device)
        c = lambda t: None if t is None else t.contiguous()  # noqa: E731
        call("mlcg_node_tmm", ptr(c(a1)), ptr(c(b1)), ptr(c(a2)), ptr(c(b2)), rows,
             NUM_FILTERS, 0, ptr(out), ptr(cs), ptr(ws), nws, stream_handle(a1.device))
        return (out, cs) if colsum else out
    out = tmm(a1, b1)
    if a2 is not None:
        out = out + tmm(a2, b2)
    return (out, a1.sum(0)) if colsum else out


def node_tmm_batch(problems, rows: int, device) -> list:
    """Several node_tmm reductions over `rows` rows in one launch pair
    (mlcg_node_tmm_batch).  problems: list of (a1, b1, a2, b2, colsum) with
    [rows, 128] fp32 contiguous tensors (a2, b2 may be None); returns, per
    problem, the [128, 128] product and (when colsum) the column sums of a1,
    as node_tmm does."""
    count = len(problems)
    _check(1 <= count <= 4, "node_tmm_batch takes 1 to 4 problems")
    outs, flat = [], []
    for a1, b1, a2, b2, colsum in problems:
        for t in (a1, b1, a2, b2):
            _check(t is None or (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()
                                 and t.dim() == 2 and t.shape == (rows, NUM_FILTERS)),
                   "node_tmm_batch operands must be contiguous [rows, 128] float32 on the GPU")
        out = torch.empty(NUM_FILTERS, NUM_FILTERS, dtype=torch.float32, device=device)
        cs = torch.empty(NUM_FILTERS, dtype=torch.float32, device=device) if colsum else None
        outs.append((out, cs) if colsum else out)
        flat += [ptr(a1), ptr(b1), ptr(a2), ptr(b2), ptr(out), ptr(cs)]
    nws = int(_lib.load().mlcg_node_tmm_batch_workspace_floats(rows, count))
    ws = torch.empty(nws, dtype=torch.float32, device=device)
    arr = (ctypes.c_void_p * len(flat))(*flat)
    call("mlcg_node_tmm_batch", arr, count, rows, NUM_FILTERS, 0, ptr(ws), nws,
         stream_handle(device))
    return outs


COPY_BATCH_MAX = 8  # jobs per mlcg_copy_batch launch


def copy_batch_ok(dsts, srcs) -> bool:
    """Whether copy_batch takes these pairs (see there)."""
    return len(dsts) == len(srcs) and all(
        d.is_cuda and s_.device == d.device and d.dtype == s_.dtype and d.shape == s_.shape
        and d.is_contiguous() and s_.is_contiguous() and d.data_ptr() % 16 == 0
        and s_.data_ptr() % 16 == 0 for d, s_ in zip(dsts, srcs))


def copy_batch(dsts, srcs) -> None:
    """dst.copy_(src) for every pair, device to device on the current stream,
    as one launch per eight pairs (mlcg_copy_batch).  Each pair: the same
    device, dtype and shape, both contiguous and 16-byte aligned, not
    overlapping; other pairs raise."""
    _check(len(dsts) == len(srcs), "copy_batch takes as many destinations as sources")
    if not dsts:
        return
    dev = dsts[0].device
    for d, s_ in zip(dsts, srcs):
        _check(d.is_cuda and s_.device == d.device == dev and d.dtype == s_.dtype
               and d.shape == s_.shape and d.is_contiguous() and s_.is_contiguous()
               and d.data_ptr() % 16 == 0 and s_.data_ptr() % 16 == 0,
               lambda: f"copy_batch: {tuple(s_.shape)} {s_.dtype} on {s_.device} -> "
                       f"{tuple(d.shape)} {d.dtype} on {d.device} needs one device, dtype "
                       "and shape, contiguous 16-byte aligned tensors")
    for k in range(0, len(dsts), COPY_BATCH_MAX):
        dd, ss = dsts[k:k + COPY_BATCH_MAX], srcs[k:k + COPY_BATCH_MAX]
        n = len(dd)
        src_arr = (ctypes.c_void_p * n)(*[t.data_ptr() for t in ss])
        dst_arr = (ctypes.c_void_p * n)(*[t.data_ptr() for t in dd])
        nbytes = (ctypes.c_int64 * n)(*[t.numel() * t.element_size() for t in dd])
        call("mlcg_copy_batch", src_arr, dst_arr, nbytes, n, stream_handle(dev))


SUM_ARRAYS_MAX = 8


def sum_arrays_ok(xs) -> bool:
    """Whether sum_arrays takes these tensors: 1..8 contiguous fp32 tensors of
    one shape on one GPU."""
    if not 1 <= len(xs) <= SUM_ARRAYS_MAX:
        return False
    x0 = xs[0]
    return all(isinstance(t, torch.Tensor) and t.is_cuda and t.device == x0.device
               and t.dtype == torch.float32 and t.shape == x0.shape and t.is_contiguous()
               for t in xs)


def sum_arrays(xs) -> torch.Tensor:
    """((0 + xs[0]) + xs[1]) + ... elementwise in one launch (mlcg_sum_arrays),
    bit-identical to adding them one by one in that order."""
    _check(sum_arrays_ok(xs), "sum_arrays takes 1 to 8 contiguous float32 tensors of one "
                              "shape on one GPU")
    out = torch.empty_like(xs[0])
    arr = (ctypes.c_void_p * len(xs))(*[t.data_ptr() for t in xs])
    call("mlcg_sum_arrays", arr, len(xs), xs[0].numel(), ptr(out), stream_handle(out.device))
    return out


def _mse_ok(x: torch.Tensor, y: torch.Tensor) -> bool:
    return (x.is_cuda and y.device == x.device and x.dtype == torch.float32
            and y.dtype == torch.float32 and x.shape == y.shape and x.numel() >= 1
            and x.is_contiguous() and y.is_contiguous())


def mse_mean(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """mean((x - y)^2) of two contiguous fp32 tensors of one shape on the GPU
    as a 0-dim tensor (mlcg_mse_mean: fixed summation order)."""
    require_device(x, y)
    _check(_mse_ok(x, y), "mse_mean takes two contiguous float32 tensors of one shape on the "
                          "same GPU")
    n = x.numel()
    loss = torch.empty((), dtype=torch.float32, device=x.device)
    nws = int(_lib.load().mlcg_mse_workspace_floats(n))
    ws = torch.empty(nws, dtype=torch.float32, device=x.device) if nws > 0 else None
    call("mlcg_mse_mean", ptr(x), ptr(y), n, ptr(loss), ptr(ws), nws, stream_handle(x.device))
    return loss


def mse_mean_backward(x: torch.Tensor, y: torch.Tensor, grad: torch.Tensor) -> torch.Tensor:
    """(2/n) (x - y) grad for the scalar upstream gradient `grad` (on the
    device), as torch's mse_loss backward evaluates it (mlcg_mse_mean_backward)."""
    require_device(x, y)
    _check(_mse_ok(x, y), "mse_mean_backward takes the forward's two tensors")
    g = grad.reshape(()).to(torch.float32).contiguous()
    out = torch.empty_like(x)
    call("mlcg_mse_mean_backward", ptr(x), ptr(y), ptr(g), x.numel(), ptr(out),
         stream_handle(x.device))
    return out


def embedding_gather(table: torch.Tensor, types: torch.Tensor) -> torch.Tensor:
    """table[types] for a [T, 128] fp32 table and int64 types (the embedding
    lookup, mlcg_embedding_gather); a type outside [0, T) gives a zero row and
    sets NUMERICS_TYPE_RANGE (check_numerics raises)."""
    require_device(table, types)
    _check(table.dim() == 2 and table.shape[1] == NUM_FILTERS and table.dtype == torch.float32,
           "embedding_gather takes a [T, 128] float32 table")
    _check(types.dtype == torch.int64 and types.dim() == 1, "types must be 1-D int64")
    t = table.contiguous()
    ty = types.contiguous()
    out = torch.empty(ty.shape[0], NUM_FILTERS, dtype=torch.float32, device=table.device)
    call("mlcg_embedding_gather", ptr(t), t.shape[0], NUM_FILTERS, ptr(ty), ty.shape[0],
         ptr(out), stream_handle(table.device))
    return out


def type_sum(x: torch.Tensor, types: torch.Tensor, num_types: int, want_bad: bool = True
             ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """(out [num_types, 128], bad [1] int32): out[t] = sum of the rows of x
    whose type is t (the embedding-table gradient), summed in a fixed order
    (mlcg_type_sum); bad[0] = 1 when a type lies outside [0, num_types).
    With want_bad=False bad is None and such a type raises bit 2 of the
    numerics flags instead (check_numerics reports it)."""
    require_device(x, types)
    _check(x.dim() == 2 and x.shape[1] == NUM_FILTERS and x.dtype == torch.float32,
           f"type_sum takes [N, {NUM_FILTERS}] float32 rows")
    _check(types.dtype == torch.int64 and types.shape == (x.shape[0],)
           and types.device == x.device, "types must be int64 [N] on the rows' device")
    _check(1 <= num_types <= 128, "type_sum supports 1..128 types")
    x, types = x.contiguous(), types.contiguous()
    out = torch.empty(num_types, NUM_FILTERS, dtype=torch.float32, device=x.device)
    bad = torch.zeros(1, dtype=torch.int32, device=x.device) if want_bad else None
    nws = int(_lib.load().mlcg_type_sum_workspace_floats(x.shape[0], num_types))
    ws = torch.empty(nws, dtype=torch.float32, device=x.device) if nws > 0 else None
    call("mlcg_type_sum", ptr(x), ptr(types), x.shape[0], NUM_FILTERS, num_types, ptr(out),
         ptr(bad), ptr(ws), nws, stream_handle(x.device))
    return out, bad


# --------------------------------------------------------------------------
# Output network MLP([128, HH, 1])

OUT_HIDDEN = (32, 64, 128)


def out_forward(x: torch.Tensor, W0: torch.Tensor, b0: Optional[torch.Tensor],
                w1: torch.Tensor, b1: Optional[torch.Tensor], act: int,
                seed: Optional[torch.Tensor] = None, reverse: bool = False,
                want_o: bool = True, save: bool = True):
    """(o [N], oz [N, HH] | None, os [N, HH] | None, xbar [N, 128] | None) of
    the output network o = act(x W0^T + b0) . w1 + b1 (mlcg_out_forward).
    With reverse, xbar = ((seed w1) * act'(oz)) W0 (seed None = ones).  oz
    is kept only for the shifted softplus (tanh derivatives need os only)."""
    require_device(x)
    hh = W0.shape[0]
    _check(x.dim() == 2 and x.shape[1] == NUM_FILTERS and x.dtype == torch.float32,
           "out_forward takes [N, 128] float32 rows")
    _check(hh in OUT_HIDDEN and tuple(W0.shape) == (hh, NUM_FILTERS) and w1.numel() == hh,
           f"unsupported output network shape {tuple(W0.shape)}")
    n = x.shape[0]
    dev = x.device
    x = x.contiguous()
    o = torch.empty(n, dtype=torch.float32, device=dev) if want_o else None
    os_ = torch.empty(n, hh, dtype=torch.float32, device=dev) if save else None
    oz = torch.empty(n, hh, dtype=torch.float32, device=dev) if save and act != 0 else None
    xbar = torch.empty_like(x) if reverse else None
    if seed is not None:
        seed = seed.contiguous().to(torch.float32)
        _check(seed.numel() == n, "seed must have one entry per node")
    call("mlcg_out_forward", ptr(x), n, NUM_FILTERS, hh, ptr(W0.contiguous()),
         ptr(None if b0 is None else b0.contiguous()), ptr(w1.contiguous().view(-1)),
         ptr(None if b1 is None else b1.contiguous()), int(act), int(reverse), ptr(seed),
         ptr(o), ptr(oz), ptr(os_), ptr(xbar), stream_handle(dev))
    return o, oz, os_, xbar


def out_rev2(x: torch.Tensor, xdot: Optional[torch.Tensor], W0: torch.Tensor,
             w1: torch.Tensor, oz: Optional[torch.Tensor], os_: torch.Tensor, act: int,
             tw: Optional[torch.Tensor], pw: Optional[torch.Tensor], has_b0: bool,
             has_b1: bool, want_odot: bool = False):
    """(odot | None, xbar2, gW0, gb0 | None, gW1 [1, HH], gb1 | None): the
    tangent and second reverse sweep of the output network (mlcg_out_rev2)."""
    require_device(x)
    hh = W0.shape[0]
    n = x.shape[0]
    dev = x.device
    c = lambda t: None if t is None else t.contiguous()  # noqa: E731
    x, xdot, oz, os_, tw, pw = map(c, (x, xdot, oz, os_, tw, pw))
    _check(os_ is not None and tuple(os_.shape) == (n, hh), "os must be [N, HH]")
    _check(xdot is None or xdot.shape == x.shape, "xdot must match x")
    _check(not want_odot or xdot is not None, "odot needs a tangent direction")
    odot = torch.empty(n, dtype=torch.float32, device=dev) if want_odot else None
    xbar2 = torch.empty_like(x)
    gW0 = torch.empty(hh, NUM_FILTERS, dtype=torch.float32, device=dev)
    gb0 = torch.empty(hh, dtype=torch.float32, device=dev) if has_b0 else None
    gW1 = torch.empty(1, hh, dtype=torch.float32, device=dev)
    gb1 = torch.empty(1, dtype=torch.float32, device=dev) if has_b1 else None
    nws = int(_lib.load().mlcg_out_rev2_workspace_floats(n, hh))
    ws = torch.empty(max(nws, 1), dtype=torch.float32, device=dev)
    call("mlcg_out_rev2", ptr(x), ptr(xdot), n, NUM_FILTERS, hh, ptr(W0.contiguous()),
         ptr(w1.contiguous().view(-1)), ptr(oz), ptr(os_), int(act), ptr(tw), ptr(pw),
         ptr(odot), ptr(xbar2), ptr(gW0), ptr(gb0), ptr(gW1), ptr(gb1), ptr(ws), nws,
         stream_handle(dev))
    return odot, xbar2, gW0, gb0, gW1, gb1


# --------------------------------------------------------------------------
# Filter network

@dataclass
class FilterSpec:
    """Description of one fused RBF -> cutoff -> MLP -> cutoff chain.

    basis 0 (Gaussian): centers = offset [K], widths = coeff [1];
    basis 1 (ExpNormal): centers = means [K], widths = betas [K], alpha.
    centers/widths are float32 device tensors the kernels read at launch
    (they may be the module's own parameters)."""

    centers: torch.Tensor
    widths: torch.Tensor
    num_rbf: int
    rbf_cut_kind: int
    rbf_lo: float
    rbf_hi: float
    conv_cut_kind: int
    conv_lo: float
    conv_hi: float
    act: int
    basis: int = 0
    alpha: float = 0.0

    def basis_args(self):
        return (int(self.basis), ptr(self.centers), ptr(self.widths), float(self.alpha))


BASIS_GAUSSIAN, BASIS_EXPNORMAL = 0, 1


FILTER_FP32, FILTER_FP16, FILTER_FP32_STRICT = 0, 1, 2


def filter_fwd(pos: torch.Tensor, graph: PairGraph, spec: FilterSpec, W1: torch.Tensor,
               b1: torch.Tensor, W2: torch.Tensor, f16: bool = False,
               want_dist: bool = True, strict_fp32: bool = False,
               out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
               ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """W [P, F], dW/dd [P, F] (fp32, or fp16 when f16) and distances [P].
    fp32 results come from split-fp16 products (about 22 significant bits
    per operand, fp32 accumulation) unless strict_fp32 asks for the fp32
    MFMA throughout (mlcg_filter_fwd's FP32_STRICT mode).  `out` = (W, Wd)
    written in place of new tensors (a caller that launches on another
    stream allocates them on the stream that consumes them)."""
    pos = _validate_pos(pos)
    F = W1.shape[0]
    _check(F == NUM_FILTERS, lambda: f"num_filters must be {NUM_FILTERS} for the HIP filter kernel")
    _check(tuple(W1.shape) == (F, spec.num_rbf) and tuple(W2.shape) == (F, F)
           and tuple(b1.shape) == (F,), "filter weights have unexpected shapes")
    cap = graph.pair_capacity
    dt = torch.float16 if f16 else torch.float32
    if out is None:
        W = torch.empty(cap, F, dtype=dt, device=pos.device)
        Wd = torch.empty(cap, F, dtype=dt, device=pos.device)
    else:
        W, Wd = out
        _check(all(t.dtype == dt and tuple(t.shape) == (cap, F) and t.is_contiguous()
                   and t.device == pos.device for t in (W, Wd)),
               "filter_fwd out tensors must be contiguous [pair_capacity, 128] of the result dtype")
    dist = torch.empty(cap, dtype=torch.float32, device=pos.device) if want_dist else None
    W1c, b1c, W2c = (t.detach().float().contiguous() for t in (W1, b1, W2))
    call("mlcg_filter_fwd", ptr(pos), ptr(graph.pair_ij), cap, ptr(graph.n_pairs_dev), cap,
         *spec.basis_args(), spec.num_rbf, spec.rbf_cut_kind, spec.rbf_lo,
         spec.rbf_hi, spec.conv_cut_kind, spec.conv_lo, spec.conv_hi, spec.act, ptr(W1c),
         ptr(b1c), ptr(W2c), F,
         FILTER_FP16 if f16 else (FILTER_FP32_STRICT if strict_fp32 else FILTER_FP32),
         ptr(W), ptr(Wd), ptr(dist), stream_handle(pos.device))
    return W, Wd, dist


NUMERICS_BWD_RANGE = 1  # mlcg_numerics_flags bit 0
NUMERICS_WEIGHT_RANGE = 2  # bit 1
NUMERICS_TYPE_RANGE = 4  # bit 2


def numerics_flags(device=None, clear: bool = True) -> torch.Tensor:
    """The split-product kernels' flag word on `device` as a one-element int32
    device tensor (no host synchronisation), cleared afterwards by default.
    Bit 0 (NUMERICS_BWD_RANGE): a filter backward met |h| or |h'| >= 2^19, so
    its weight gradients may be non-finite.  Bit 1 (NUMERICS_WEIGHT_RANGE): a
    split filter kernel met a weight >= 65504 (the fp16 maximum) in magnitude.
    Bit 2 (NUMERICS_TYPE_RANGE): embedding_gather met a type outside its table."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    call("mlcg_numerics_flags", ptr(out), int(clear), stream_handle(dev))
    return out


def check_numerics(device=None) -> None:
    """Raise RuntimeError if a split-product kernel reported a value past its
    range since the last check (one host synchronisation); clears the flags."""
    v = int(numerics_flags(device, clear=True).item())
    if v & NUMERICS_TYPE_RANGE:
        raise RuntimeError("embedding lookup: an atom type lies outside the embedding table "
                           "(its row was set to zero)")
    if v & NUMERICS_WEIGHT_RANGE:
        raise RuntimeError(
            "filter kernels: a filter weight reached 65504 (the fp16 maximum) or more in "
            "magnitude, past the range of the split-fp16 products; filters and their gradients may be non-finite. "
            "Use strict fp32 filters (model.strict_fp32_filters = True) for such models")
    if v & NUMERICS_BWD_RANGE:
        raise RuntimeError(
            "filter backward: an activation value or derivative reached 2^19 or more, past "
            "the range of the split-fp16 products; weight gradients may be non-finite. "
            "Use strict fp32 filters (model.strict_fp32_filters = True) for such models")


def _pair_adjoint_outputs(want: bool, cap: int, F: int, dev):
    if not want:
        return None, None
    return (torch.empty(cap, F, dtype=torch.float32, device=dev),
            torch.empty(cap, F, dtype=torch.float32, device=dev))


def filter_bwd(pos: torch.Tensor, graph: PairGraph, spec: FilterSpec, W1: torch.Tensor,
               b1: torch.Tensor, W2: torch.Tensor, Wbar: torch.Tensor,
               Wdbar: torch.Tensor, pair_adjoints: bool = False, strict_fp32: bool = False):
    """Gradients (dW1 [F, K], db1 [F], dW2 [F, F]) of <Wbar, W> + <Wdbar, dW/dd>;
    with pair_adjoints also the first-layer pair adjoints (abar, adbar)
    [P, F] that rbf_param_grad consumes.  strict_fp32 runs every product on
    the fp32 MFMA instead of split-fp16 products (which hold activations and
    derivatives below 2^19, see check_numerics)."""
    pos = _validate_pos(pos)
    F = W1.shape[0]
    K = spec.num_rbf
    cap = graph.pair_capacity
    dev = pos.device
    _check(tuple(Wbar.shape) == (cap, F) and tuple(Wdbar.shape) == (cap, F),
           "Wbar / Wdbar must be [pair_capacity, F]")
    nws = int(_lib.load().mlcg_filter_bwd_workspace_floats(cap, K))
    _check(nws > 0, lambda: f"num_rbf={K} is not supported by the filter backward")
    ws = torch.empty(nws, dtype=torch.float32, device=dev)
    dW1 = torch.empty(F, K, dtype=torch.float32, device=dev)
    db1 = torch.empty(F, dtype=torch.float32, device=dev)
    dW2 = torch.empty(F, F, dtype=torch.float32, device=dev)
    W1c, b1c, W2c = (t.detach().float().contiguous() for t in (W1, b1, W2))
    ab, adb = _pair_adjoint_outputs(pair_adjoints, cap, F, dev)
    call("mlcg_filter_bwd", ptr(pos), ptr(graph.pair_ij), cap, ptr(graph.n_pairs_dev), cap,
         *spec.basis_args(), K, spec.rbf_cut_kind, spec.rbf_lo, spec.rbf_hi,
         spec.conv_cut_kind, spec.conv_lo, spec.conv_hi, spec.act, ptr(W1c), ptr(b1c),
         ptr(W2c), F, ptr(Wbar.contiguous()), ptr(Wdbar.contiguous()), ptr(dW1), ptr(db1),
         ptr(dW2), ptr(ab), ptr(adb), ptr(ws), nws, int(strict_fp32), stream_handle(dev))
    if pair_adjoints:
        return dW1, db1, dW2, ab, adb
    return dW1, db1, dW2


def filter_bwd_cfconv(pos: torch.Tensor, graph: PairGraph, spec: FilterSpec,
                      W1: torch.Tensor, b1: torch.Tensor, W2: torch.Tensor,
                      gagg2: torch.Tensor, y: torch.Tensor, gagg1: Optional[torch.Tensor],
                      ydot: Optional[torch.Tensor],
                      ddot: Optional[torch.Tensor], pair_adjoints: bool = False,
                      strict_fp32: bool = False):
    """filter_bwd with Wbar_p = g2_i y_j + g2_j y_i + g1_i yd_j + g1_j yd_i and
    Wdbar_p = dd_p (g1_i y_j + g1_j y_i) formed in the kernel from node arrays
    (pair_adjoints and strict_fp32 as in filter_bwd)."""
    pos = _validate_pos(pos)
    F = W1.shape[0]
    K = spec.num_rbf
    cap = graph.pair_capacity
    dev = pos.device
    nws = int(_lib.load().mlcg_filter_bwd_workspace_floats(cap, K))
    _check(nws > 0, lambda: f"num_rbf={K} is not supported by the filter backward")
    ws = torch.empty(nws, dtype=torch.float32, device=dev)
    dW1 = torch.empty(F, K, dtype=torch.float32, device=dev)
    db1 = torch.empty(F, dtype=torch.float32, device=dev)
    dW2 = torch.empty(F, F, dtype=torch.float32, device=dev)
    W1c, b1c, W2c = (t.detach().float().contiguous() for t in (W1, b1, W2))
    c = lambda t: None if t is None else t.contiguous()  # noqa: E731
    ab, adb = _pair_adjoint_outputs(pair_adjoints, cap, F, dev)
    call("mlcg_filter_bwd_cfconv", ptr(pos), ptr(graph.pair_ij), cap, ptr(graph.n_pairs_dev),
         cap, *spec.basis_args(), K, spec.rbf_cut_kind, spec.rbf_lo, spec.rbf_hi,
         spec.conv_cut_kind, spec.conv_lo, spec.conv_hi, spec.act, ptr(W1c), ptr(b1c),
         ptr(W2c), F, ptr(c(gagg2)), ptr(c(y)), ptr(c(gagg1)), ptr(c(ydot)), ptr(ddot),
         ptr(dW1), ptr(db1), ptr(dW2), ptr(ab), ptr(adb), ptr(ws), nws, int(strict_fp32),
         stream_handle(dev))
    if pair_adjoints:
        return dW1, db1, dW2, ab, adb
    return dW1, db1, dW2


def rbf_param_grad(dist: torch.Tensor, graph: PairGraph, spec: FilterSpec, W1: torch.Tensor,
                   abar: torch.Tensor, adbar: torch.Tensor,
                   out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
    """(dcenters [K], dwidths [K]) of the basis from the first-layer pair
    adjoints (mlcg_rbf_param_grad); added into `out` when given."""
    require_device(dist, abar, adbar)
    K = spec.num_rbf
    cap = graph.pair_capacity
    dev = dist.device
    _check(tuple(abar.shape) == (cap, NUM_FILTERS) and abar.shape == adbar.shape,
           "abar / adbar must be [pair_capacity, F]")
    nws = int(_lib.load().mlcg_rbf_param_grad_workspace_floats(cap, K))
    _check(nws > 0, lambda: f"num_rbf={K} is not supported")
    ws = torch.empty(nws, dtype=torch.float32, device=dev)
    accumulate = out is not None
    if out is None:
        out = (torch.empty(K, dtype=torch.float32, device=dev),
               torch.empty(K, dtype=torch.float32, device=dev))
    W1c = W1.detach().float().contiguous()
    call("mlcg_rbf_param_grad", ptr(dist), ptr(graph.n_pairs_dev), cap, *spec.basis_args(), K,
         spec.rbf_cut_kind, spec.rbf_lo, spec.rbf_hi, ptr(W1c), NUM_FILTERS,
         ptr(abar.contiguous()), ptr(adbar.contiguous()), int(accumulate), ptr(out[0]),
         ptr(out[1]), ptr(ws), nws, stream_handle(dev))
    return out


# --------------------------------------------------------------------------
# CFConv gather/scatter family

def _wptr(W: torch.Tensor) -> Tuple[int, int]:
    return ptr(W), int(W.dtype == torch.float16)


def cfconv_gather(src: torch.Tensor, W: torch.Tensor, graph: PairGraph) -> torch.Tensor:
    """out[i] = sum_j src[j] * W[p(i, j)]  (schnet.py:346,368).  float64 src
    and W (a model moved to double) take mlcg_cfconv_gather_f64, any width."""
    require_device(src, W)
    src = src.contiguous()
    out = torch.empty_like(src)
    if src.dtype == torch.float64:
        _check(W.dtype == torch.float64 and W.shape[1] == src.shape[1],
               "a float64 gather takes float64 filters of the source's width")
        call("mlcg_cfconv_gather_f64", ptr(src), ptr(W.contiguous()), ptr(graph.rowptr),
             ptr(graph.col), ptr(graph.eid2pair), graph.num_nodes, src.shape[1], ptr(out),
             stream_handle(src.device))
        return out
    wp, wf16 = _wptr(W)
    call("mlcg_cfconv_gather", ptr(src), wp, wf16, ptr(graph.rowptr), ptr(graph.col),
         ptr(graph.eid2pair), graph.num_nodes, src.shape[1], ptr(out),
         stream_handle(src.device))
    return out


def cfconv_gather_bwd(gagg: torch.Tensor, y: torch.Tensor, W: torch.Tensor, Wd: torch.Tensor,
                      graph: PairGraph, dbar: torch.Tensor, accumulate: bool = True,
                      want_ybar: bool = True) -> Optional[torch.Tensor]:
    """ybar = gather(gagg, W); dbar[p] += <Wd_p, gagg_i y_j + gagg_j y_i> in
    place (dbar[p] = ... with accumulate=False: dbar may be uninitialised).
    want_ybar=False: dbar only (the same values), returns None."""
    gagg = gagg.contiguous()
    ybar = torch.empty_like(gagg) if want_ybar else None
    wp, wf16 = _wptr(W)
    call("mlcg_cfconv_gather_bwd", ptr(gagg), ptr(y.contiguous()), wp, ptr(Wd), wf16,
         ptr(graph.rowptr), ptr(graph.col), ptr(graph.eid2pair), graph.num_nodes,
         gagg.shape[1], ptr(ybar), ptr(dbar), int(accumulate), stream_handle(gagg.device))
    return ybar


def cfconv_gather_tangent(ydot: Optional[torch.Tensor], y: torch.Tensor, W: torch.Tensor,
                          Wd: torch.Tensor, ddot: torch.Tensor, graph: PairGraph) -> torch.Tensor:
    y = y.contiguous()
    out = torch.empty_like(y)
    call("mlcg_cfconv_gather_tangent", ptr(None if ydot is None else ydot.contiguous()),
         ptr(y), ptr(W), ptr(Wd), ptr(ddot), ptr(graph.rowptr), ptr(graph.col),
         ptr(graph.eid2pair), graph.num_nodes, y.shape[1], ptr(out), stream_handle(y.device))
    return out


def cfconv_gather_rev2(gagg2: torch.Tensor, gagg1: Optional[torch.Tensor], y: torch.Tensor,
                       ydot: Optional[torch.Tensor], W: torch.Tensor, Wd: torch.Tensor,
                       ddot: Optional[torch.Tensor], graph: PairGraph,
                       pair_adjoints: bool = True):
    """ybar2 and (with pair_adjoints) the [P, F] adjoints Wbar, Wdbar."""
    gagg2 = gagg2.contiguous()
    F = gagg2.shape[1]
    ybar2 = torch.empty_like(gagg2)
    cap = graph.pair_capacity
    Wbar = Wdbar = None
    if pair_adjoints:
        Wbar = torch.empty(cap, F, dtype=torch.float32, device=gagg2.device)
        Wdbar = torch.empty(cap, F, dtype=torch.float32, device=gagg2.device)
    call("mlcg_cfconv_gather_rev2", ptr(gagg2),
         ptr(None if gagg1 is None else gagg1.contiguous()), ptr(y.contiguous()),
         ptr(None if ydot is None else ydot.contiguous()), ptr(W), ptr(Wd), ptr(ddot),
         ptr(graph.rowptr), ptr(graph.col), ptr(graph.eid2pair), graph.num_nodes, F,
         ptr(ybar2), ptr(Wbar), ptr(Wdbar), stream_handle(gagg2.device))
    return ybar2, Wbar, Wdbar


def pair_ddot(pos: torch.Tensor, dist: torch.Tensor, graph: PairGraph,
              u: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """ddot[p] = scale * rhat_p . (u[j] - u[i]) over the graph's pairs."""
    cap = graph.pair_capacity
    ddot = torch.empty(cap, dtype=torch.float32, device=pos.device)
    call("mlcg_pair_ddot", ptr(pos), ptr(dist), ptr(graph.pair_ij), cap,
         ptr(graph.n_pairs_dev), cap, ptr(u.contiguous()), float(scale), ptr(ddot),
         stream_handle(pos.device))
    return ddot


def pair_forces(pos: torch.Tensor, dist: torch.Tensor, dbar: torch.Tensor,
                graph: PairGraph, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """F_i = sum_j dbar[p(i,j)] (pos_j - pos_i) / d  (= -dE/dpos_i)."""
    accumulate = out is not None
    if out is None:
        out = torch.empty_like(pos)
    call("mlcg_pair_forces", ptr(pos), ptr(dist), ptr(dbar), ptr(graph.rowptr),
         ptr(graph.col), ptr(graph.eid2pair), graph.num_nodes, int(accumulate), ptr(out),
         stream_handle(pos.device))
    return out


def segment_sum(values: torch.Tensor, frame_ptr: torch.Tensor) -> torch.Tensor:
    """Per-frame sums of a [N] or [N, 1] float32 (or float64) vector."""
    require_device(values)
    v = values.contiguous().view(-1)
    nb = frame_ptr.numel() - 1
    if v.dtype == torch.float64:
        out = torch.empty(nb, dtype=torch.float64, device=values.device)
        call("mlcg_segment_sum_f64", ptr(v), ptr(frame_ptr), nb, ptr(out),
             stream_handle(values.device))
        return out
    out = torch.empty(nb, dtype=torch.float32, device=values.device)
    call("mlcg_segment_sum", ptr(v), 1, ptr(frame_ptr), nb, ptr(out),
         stream_handle(values.device))
    return out


# --------------------------------------------------------------------------
# Priors

PRIOR_KIND = {"bonds": 0, "angles": 1, "dihedrals": 2, "repulsion": 3}
PRIOR_ORDER = {0: 2, 1: 3, 2: 4, 3: 2}


@dataclass
class PriorGraph:
    """Interaction list of one prior plus the index structures its kernels use.

    index_mapping : [order, M] int64 (bead of slot s of interaction m)
    bead_ptr      : [N + 1] int32 CSR over bead_slots
    bead_slots    : [M * order] int32 flat slot ids m * order + s, grouped by
                    bead and ascending within a bead
    seg_ptr       : [B + 1] int64, interactions of frame b are
                    seg_ptr[b] : seg_ptr[b + 1] (mapping_batch is sorted)
    pair_records  : (params, params version, int32 records) -- the bead-major
                    slot records and bead windows of the direct repulsion
                    path, made for that parameter matrix (prior_pair_records)
    """

    index_mapping: torch.Tensor
    bead_ptr: torch.Tensor
    bead_slots: torch.Tensor
    seg_ptr: torch.Tensor
    num_nodes: int
    num_frames: int
    pair_records: Optional[tuple] = None

    @property
    def num_interactions(self) -> int:
        return self.index_mapping.shape[1]


def prior_graph(index_mapping: torch.Tensor, mapping_batch: Optional[torch.Tensor],
                num_nodes: int, num_frames: int) -> PriorGraph:
    """Builds the bead -> slot CSR and the frame segments of an interaction
    list (once per topology; the MD loop reuses it every step)."""
    require_device(index_mapping)
    _check(index_mapping.dim() == 2 and index_mapping.shape[0] in (2, 3, 4),
           f"index_mapping must be [order, M], got {tuple(index_mapping.shape)}")
    im = _as_i64(index_mapping)
    order, M = im.shape
    dev = im.device
    if M > 0:
        _check(int(im.min()) >= 0 and int(im.max()) < num_nodes,
               "index_mapping refers to beads outside [0, num_nodes)")
    flat = im.t().reshape(-1)  # slot id m * order + s -> bead
    srt = torch.sort(flat, stable=True)
    bead_slots = srt.indices.to(torch.int32).contiguous()
    counts = torch.bincount(flat, minlength=num_nodes)
    bead_ptr = torch.zeros(num_nodes + 1, dtype=torch.int32, device=dev)
    bead_ptr[1:] = torch.cumsum(counts, 0).to(torch.int32)
    if mapping_batch is None:
        mapping_batch = torch.zeros(M, dtype=torch.int64, device=dev)
    mb = _as_i64(mapping_batch)
    _check(mb.numel() == M, "mapping_batch must have one entry per interaction")
    if M > 1:
        _check(bool((mb[1:] >= mb[:-1]).all()),
               "mapping_batch must be sorted by frame (collated neighbour lists are)")
    seg_ptr = frame_ptr_from_batch(mb, num_frames)
    return PriorGraph(index_mapping=im, bead_ptr=bead_ptr, bead_slots=bead_slots,
                      seg_ptr=seg_ptr, num_nodes=num_nodes, num_frames=num_frames)


def prior_terms(kind: int, n_degs: int, pos: torch.Tensor, graph: PriorGraph,
                params: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(energy [M], slot forces [M, order, 3]) of every interaction, in the
    positions' type (float32, or float64 for a model moved to double)."""
    f64 = pos.dtype == torch.float64
    pos = _validate_pos_f64(pos) if f64 else _validate_pos(pos)
    dt = pos.dtype
    M = graph.num_interactions
    order = PRIOR_ORDER[kind]
    n_params = int(_lib.load().mlcg_prior_num_params(kind, n_degs))
    params = params.to(dt).contiguous()
    _check(tuple(params.shape) == (M, n_params),
           f"params must be [{M}, {n_params}], got {tuple(params.shape)}")
    energy = torch.empty(M, dtype=dt, device=pos.device)
    slot_f = torch.empty(M, order, 3, dtype=dt, device=pos.device)
    call("mlcg_prior_terms_f64" if f64 else "mlcg_prior_terms", kind, n_degs, ptr(pos),
         ptr(graph.index_mapping), M, M, ptr(params), n_params, ptr(energy), ptr(slot_f),
         stream_handle(pos.device))
    return energy, slot_f


def _validate_pos_f64(pos: torch.Tensor) -> torch.Tensor:
    require_device(pos)
    _check(pos.dim() == 2 and pos.shape[1] == 3, lambda: f"pos must be [N, 3], got {tuple(pos.shape)}")
    return pos.contiguous()


def prior_pair_records(graph: PriorGraph, params: torch.Tensor) -> torch.Tensor:
    """int32 records of the direct repulsion path (mlcg_prior_pair_records:
    bead-major {partner | role << 31, sigma} per slot and the bead windows the
    kernels stage), cached on the graph for the parameter matrix they were
    made from (the same tensor at the same version: the prior modules hand
    out one cached matrix per topology)."""
    c = graph.pair_records
    if c is not None and c[0] is params and c[1] == params._version:
        return c[2]
    M, n = graph.num_interactions, graph.num_nodes
    size = int(_lib.load().mlcg_prior_pair_records_ints(n, M))
    rec = torch.empty(size, dtype=torch.int32, device=params.device)
    call("mlcg_prior_pair_records", ptr(graph.index_mapping), M, M, ptr(params),
         params.shape[1], ptr(graph.bead_ptr), ptr(graph.bead_slots), n, ptr(rec),
         stream_handle(params.device))
    graph.pair_records = (params, params._version, rec)
    return rec


def prior_energy_forces(kind: int, n_degs: int, pos: torch.Tensor, graph: PriorGraph,
                        params: torch.Tensor, forces: Optional[torch.Tensor] = None):
    """Per-frame energies [B] and forces [N, 3] of one prior; with `forces`
    given the forces are added to it in place.  The repulsion prior takes its
    forces straight from the positions per bead (mlcg_prior_repulsion, the
    same values as the slot-force path, without slot force arrays)."""
    accumulate = forces is not None
    f64 = pos.dtype == torch.float64
    if forces is None:
        forces = torch.empty(graph.num_nodes, 3, dtype=pos.dtype if f64 else torch.float32,
                             device=pos.device)
    if kind == PRIOR_KIND["repulsion"] and not f64:
        pos = _validate_pos(pos)
        M = graph.num_interactions
        params = params.to(torch.float32).contiguous()
        _check(tuple(params.shape) == (M, 1), f"params must be [{M}, 1], got {tuple(params.shape)}")
        _check(pos.shape[0] == graph.num_nodes,
               "pos must hold the prior graph's num_nodes beads")
        rec = prior_pair_records(graph, params)
        energy = torch.empty(M, dtype=torch.float32, device=pos.device)
        call("mlcg_prior_repulsion", ptr(pos), graph.num_nodes, ptr(graph.index_mapping), M, M,
             ptr(params), ptr(rec), ptr(graph.bead_ptr), ptr(energy), int(accumulate),
             ptr(forces), stream_handle(pos.device))
        return segment_sum(energy, graph.seg_ptr), forces
    energy, slot_f = prior_terms(kind, n_degs, pos, graph, params)
    E = segment_sum(energy, graph.seg_ptr)
    _check(forces.dtype == energy.dtype, "forces must have the positions' dtype")
    call("mlcg_prior_gather_forces_f64" if f64 else "mlcg_prior_gather_forces", ptr(slot_f),
         ptr(graph.bead_ptr), ptr(graph.bead_slots), graph.num_nodes, int(accumulate),
         ptr(forces), stream_handle(pos.device))
    return E, forces


# --------------------------------------------------------------------------
# Langevin BAOAB

def langevin_baoa(pos: torch.Tensor, vel: torch.Tensor, forces: torch.Tensor,
                  masses: torch.Tensor, beta_mass_ratio: torch.Tensor, dt: float,
                  vscale: float, noisescale: float, seed: int,
                  step: Optional[torch.Tensor] = None,
                  noise: Optional[torch.Tensor] = None) -> None:
    """B, A, O, A sub-steps in place on pos and vel ([N, 3] float32, or all
    float64 for a simulation in double precision)."""
    require_device(pos, vel, forces, masses, beta_mass_ratio)
    dt_ = pos.dtype if pos.dtype == torch.float64 else torch.float32
    for t in (pos, vel, forces):
        _check(t.dtype == dt_ and t.is_contiguous() and t.shape == pos.shape,
               f"pos, vel and forces must be contiguous {dt_} [N, 3]")
    n = pos.shape[0]
    _check(masses.numel() == n and beta_mass_ratio.numel() == n,
           "masses and beta_mass_ratio must have one entry per bead")
    if noise is not None:
        _check(noise.shape == pos.shape and noise.dtype == dt_, f"noise must be {dt_} [N, 3]")
        noise = noise.contiguous()
    if step is not None:
        _check(step.dtype == torch.int64 and step.numel() == 1, "step must be one int64")
    call("mlcg_langevin_baoa_f64" if dt_ == torch.float64 else "mlcg_langevin_baoa", ptr(pos),
         ptr(vel), ptr(forces), ptr(masses.to(dt_).contiguous()),
         ptr(beta_mass_ratio.to(dt_).contiguous()), n, float(dt), float(vscale),
         float(noisescale), int(seed) & ((1 << 64) - 1), ptr(step), ptr(noise),
         stream_handle(pos.device))


def langevin_b(vel: torch.Tensor, forces: torch.Tensor, masses: torch.Tensor, dt: float,
               step: Optional[torch.Tensor] = None) -> None:
    """Final B sub-step in place on vel; advances `step` by one."""
    require_device(vel, forces, masses)
    if vel.dtype == torch.float64:
        _check(forces.dtype == torch.float64, "forces must be float64 with float64 velocities")
        call("mlcg_langevin_b_f64", ptr(vel), ptr(forces),
             ptr(masses.to(torch.float64).contiguous()), vel.shape[0], float(dt), ptr(step),
             stream_handle(vel.device))
        return
    call("mlcg_langevin_b", ptr(vel), ptr(forces), ptr(masses.to(torch.float32).contiguous()),
         vel.shape[0], float(dt), ptr(step), stream_handle(vel.device))


def philox_normals(seed: int, step: int, n: int, device) -> torch.Tensor:
    """The [n, 3] normals langevin_baoa draws at `step` (for statistics tests)."""
    out = torch.empty(n, 3, dtype=torch.float32, device=device)
    call("mlcg_philox_normals", int(seed) & ((1 << 64) - 1), int(step), n, ptr(out),
         stream_handle(torch.device(device)))
    return out
