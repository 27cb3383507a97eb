#!/usr/bin/env python
"""Benchmark of the SchNet CFConv hot path on one MI355X.

Workload: full SchNet CG model -- embedding 128, three
interaction blocks, 50 Gaussian RBF on 0-20 A with a cosine envelope, cosine
cutoff 20 A, output MLP 128 -> 64 -> 1, Tanh -- on 512 frames of a 35-bead
self-avoiding chain, synthetic and seeded (``mlcg_amd.synthetic.config2``),
random-init weights.  One step is the reference's force-matching training
step (mlcg/pl/model.py:113-131 plus Lightning's backward and AdamW step):

    radius graph -> energies -> forces (create_graph) -> ForceMSE ->
    double backward to every parameter -> AdamW.step()

Metric: CFConv edges/s := E_directed * n_blocks / t_step (forward + force +
double backward of every block per step), with the inputs resident in HBM.
The headline step runs through mlcg_amd.pl.CapturedTrainStep: the whole step
recorded once as a HIP graph, each timed step loading its batch into the
recorded inputs (one batched device copy, mlcg_copy_batch) and replaying the
graph, so the figure does not depend on how fast the host issues ~140
launches.  The
same step issued eagerly from Python is timed beside it (`eager_step`, with
the host's issue time per step and the device time of a step queued ahead).

Besides the JSON contract fields the line carries
  roofline      -- the dominant HIP kernel (by device time over the timed
                   steps, launches bracketed by HIP events on the launch
                   stream): algorithmic bytes or FLOPs per launch / average
                   launch time, against the MI355X peak;
  kernels       -- the same figures for every HIP kernel of the step;
  radius_graph  -- config 3 (2048 x 100-bead globules, 15 A): edges/s of the
                   HIP radius graph, inputs resident;
  fp16_config4  -- config 4 (256 x 500 beads, fp16 filter linears): energy +
                   forces per call, and the fp16 filter kernel's MFMA fraction;
  eager_step    -- the same config-2 step launched kernel by kernel: wall
                   time, host issue time, device time, and the device time
                   with the filter forwards issued in block order;
  md_config5    -- config 5 (100 x 268-bead Langevin replicas, SchNet +
                   priors, captured step): MD steps/s;
  cpu_baseline  -- the CPU restatement (oracle/schnet_ref.py) of the same
                   step on a bounded sample of frames, host threads stated.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix
FP16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 matrix

K_RBF = 50
F = 128
H = 128
N_BLOCKS = 3
RC = 20.0


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--frames", type=int, default=512, help="config-2 frames per step")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-radius", action="store_true", help="skip the config-3 radius leg")
    p.add_argument("--no-fp16", action="store_true", help="skip the config-4 fp16 leg")
    p.add_argument("--no-md", action="store_true", help="skip the config-5 MD leg")
    p.add_argument("--gather-probe", action="store_true",
                   help="run the gather access-pattern probe (cold caches)")
    p.add_argument("--mfma-probe", action="store_true",
                   help="run the MFMA-loop probe (sustained matrix-core rate per shape)")
    p.add_argument("--stream-probe", action="store_true",
                   help="measure the HBM read / copy ceiling with the library's streaming "
                        "kernels")
    p.add_argument("--only-probes", action="store_true",
                   help="run only the requested probes (no config legs)")
    p.add_argument("--no-capture", action="store_true",
                   help="skip the captured (HIP graph) config-2 step")
    p.add_argument("--captured-only", action="store_true",
                   help="run only the captured config-2 step (for kernel traces of the "
                        "graph replays)")
    p.add_argument("--md-steps", type=int, default=200, help="MD steps of the config-5 leg")
    p.add_argument("--cpu-frames", type=int, default=32,
                   help="frames in the CPU baseline sample")
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="approximate CPU time budget of the baseline leg")
    p.add_argument("--exact-graph", action="store_true",
                   help="size the radius graph exactly each step (one host sync per step) "
                        "instead of the fixed-capacity form")
    p.add_argument("--calib-copy-mib", type=int, default=0,
                   help="run one device-to-device copy of this many MiB first (a "
                        "known-size reference dispatch for HBM byte counters)")
    return p.parse_args(argv)


# ---------------------------------------------------------------------------
# algorithmic work per launch of each HIP entry point

def algorithmic_work(name: str, E: int, P: int, N: int, B: int, f16: bool = False):
    """(bound, amount, unit) per launch: bytes for HBM-bound kernels, FLOPs
    for the MFMA filter kernels.  Minimum work only: K is not padded,
    recomputation is not counted, W is read once per unordered pair."""
    sw = 2 if f16 else 4
    kf_ff = K_RBF * F + F * F
    if name == "mlcg_filter_fwd":
        # value and distance-tangent through both linears
        return "mfma", 2 * 2 * kf_ff * P, "flop"
    if name in ("mlcg_filter_bwd", "mlcg_filter_bwd_cfconv"):
        # two reverse products through W2^T plus the pair reductions of the
        # weight gradients dW2 (two streams) and dW1 (two streams); the
        # forward recomputation of a, a' is not algorithmic work
        return "mfma", (2 * 2 * F * F + 2 * 2 * F * F + 2 * 2 * K_RBF * F) * P, "flop"
    if name == "mlcg_node_gemm":
        # one [N, 128] x [128, 128] product whose epilogue streams 2-6 [N, 128]
        # tensors: HBM-bound (at most ~32 FLOP/B against the ~104 FLOP/B
        # ridge of the split-fp16 MFMA); the wrapper reports each launch's
        # bytes, this is the plain form's
        return "hbm", 2 * 4 * F * N + 4 * (F + 1) * F, "byte"
    if name == "mlcg_node_gemm2":
        # two consecutive products in one kernel (bytes reported per launch
        # by the wrapper; this is the smallest form's: x in, two outputs)
        return "hbm", 3 * 4 * F * N + 2 * 4 * (F + 1) * F, "byte"
    if name == "mlcg_type_sum":
        # the rows of x and their types read once
        return "hbm", 4 * F * N + 8 * N, "byte"
    if name == "mlcg_cfconv_gather":
        return "hbm", sw * F * P + 4 * E + 4 * (N + 1) + 2 * 4 * F * N, "byte"
    if name == "mlcg_cfconv_gather_bwd":
        # W and Wd read, dbar RMW per pair, gagg and y in, ybar out
        return "hbm", 2 * sw * F * P + 8 * P + 4 * E + 4 * (N + 1) + 3 * 4 * F * N, "byte"
    if name == "mlcg_cfconv_gather_tangent":
        # W, Wd, ddot per pair; ydot, y in, out
        return "hbm", 2 * sw * F * P + 4 * P + 4 * E + 4 * (N + 1) + 3 * 4 * F * N, "byte"
    if name == "mlcg_cfconv_gather_rev2":
        # the fused step calls it without pair-adjoint outputs: W, Wd, ddot
        # per pair; gagg2, gagg1 in, ybar2 out
        return "hbm", 2 * sw * F * P + 4 * P + 4 * E + 4 * (N + 1) + 3 * 4 * F * N, "byte"
    # radius graph: positions, batch and frame_ptr in; CSR (rowptr, and
    # pairptr when the pair structures are built, P > 0) and the int64 edge
    # list out, with col, the pair list and its edge map when P > 0
    csr = 4 * (N + 1) * (2 if P else 1)
    pair_out = 4 * E + 12 * P if P else 0
    if name == "mlcg_radius_count":
        return "hbm", 12 * N + 8 * N + 8 * (B + 1) + 8 * N, "byte"
    if name == "mlcg_radius_rowptr":
        return "hbm", 12 * N + 8 * N + 8 * (B + 1) + csr, "byte"
    if name in ("mlcg_radius_fill", "mlcg_radius_graph"):
        return "hbm", 12 * N + 8 * N + 8 * (B + 1) + csr + 16 * E + pair_out, "byte"
    if name == "mlcg_pair_forces":
        return "hbm", 12 * N + 8 * P + 8 * E + 4 * (N + 1) + 12 * N, "byte"
    if name == "mlcg_pair_ddot":
        return "hbm", 8 * P + 4 * P + 24 * N + 4 * P, "byte"
    if name == "mlcg_pair_reverse_map":
        return "hbm", 8 * P + 4 * P + 4 * (N + 1), "byte"
    return None


# Entry points whose counted fp32 products run on the fp16 MFMA as three
# products of split operands: their MFMA ceiling, in fp32-equivalent FLOP/s,
# is a third of the fp16 peak.  (The filter backward's recomputation of the
# first layer stays on the fp32 MFMA but is not counted as algorithmic work.)
SPLIT_FP16 = {"mlcg_filter_fwd", "mlcg_filter_bwd", "mlcg_filter_bwd_cfconv"}
SPLIT_FP16_PEAK_TFLOPS = FP16_MFMA_PEAK_TFLOPS / 3

# entry point -> kernel symbol(s) it launches (as rocprofv3 names them)
KERNEL_SYMBOL = {
    "mlcg_filter_fwd": "filter_fwd_x3_kernel",
    "mlcg_filter_bwd": "filter_bwd_fused_kernel",
    "mlcg_filter_bwd_cfconv": "filter_bwd_fused_kernel",
    "mlcg_node_tmm": "node_tmm_kernel",
    "mlcg_node_gemm": "node_gemm_kernel",
    "mlcg_node_gemm2": "node_gemm2_kernel",
    "mlcg_type_sum": "type_sum_kernel",
    "mlcg_cfconv_gather": "gather_kernel",
    "mlcg_cfconv_gather_bwd": "gather_bwd_kernel",
    "mlcg_cfconv_gather_tangent": "gather_tangent_kernel",
    "mlcg_cfconv_gather_rev2": "gather_rev2_kernel",
    "mlcg_radius_count": "radius_count_kernel",
    "mlcg_radius_rowptr": "radius_rows_kernel<0, ...>",
    "mlcg_radius_fill": "radius_rows_kernel<1, ...>",
    "mlcg_radius_graph": "radius_rows_kernel<2, ...>",
    "mlcg_pair_forces": "pair_forces_kernel",
    "mlcg_pair_ddot": "pair_ddot_kernel",
    "mlcg_pair_reverse_map": "pair_reverse_kernel",
}


def kernel_report(summary, E, P, N, B, work=None):
    """Per entry point: launches, average device time and the roofline
    fraction of its algorithmic work.  `work` holds the summed work of the
    launches whose wrapper reported it (the node GEMMs' bytes, which depend
    on the epilogue); the other entry points use algorithmic_work."""
    work = work or {}
    rows = {}
    for name, (launches, total_ms) in summary.items():
        w = algorithmic_work(name, E, P, N, B)
        if w is not None and name in work:
            w = (w[0], work[name] / max(launches, 1), w[2])
        avg_ms = total_ms / max(launches, 1)
        row = {"kernel": KERNEL_SYMBOL.get(name, name), "launches": launches,
               "avg_us": round(avg_ms * 1e3, 3), "total_ms": round(total_ms, 4)}
        if w is not None:
            bound, amount, unit = w
            if bound == "hbm":
                ach = amount / (avg_ms * 1e-3) / 1e9
                row.update(bound="hbm", achieved=round(ach, 2), peak=HBM_PEAK_GBS,
                           unit="GB/s", frac=round(ach / HBM_PEAK_GBS, 4),
                           algorithmic_bytes=int(amount))
            else:
                ach = amount / (avg_ms * 1e-3) / 1e12
                split = name in SPLIT_FP16
                peak = SPLIT_FP16_PEAK_TFLOPS if split else FP32_MFMA_PEAK_TFLOPS
                row.update(bound="mfma", achieved=round(ach, 3), peak=round(peak, 1),
                           unit="TFLOP/s", frac=round(ach / peak, 4),
                           algorithmic_flops=int(amount),
                           mfma="fp16 x3 (split fp32 operands)" if split else "fp32")
        rows[name] = row
    return rows


def load_traffic(kernel_symbol: str):
    """HBM bytes per launch of `kernel_symbol` from the committed rocprofv3
    counter summary (profiles/traffic_config2.txt: lines
    `<kernel> <bytes_per_launch>`), or None when absent."""
    path = os.path.join(ROOT, "profiles", "traffic_config2.txt")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        for line in fh:
            parts = line.split()
            if len(parts) >= 2 and parts[0] == kernel_symbol and not line.startswith("#"):
                try:
                    return int(float(parts[1]))
                except ValueError:
                    return None
    return None


# ---------------------------------------------------------------------------

def build_model(torch, nn, device):
    act = torch.nn.Tanh()
    rbf = nn.GaussianBasis(nn.CosineCutoff(0.0, RC), num_rbf=K_RBF)
    model = nn.StandardSchNet(rbf, nn.CosineCutoff(0.0, RC), [64], hidden_channels=H,
                              embedding_size=100, num_filters=F,
                              num_interactions=N_BLOCKS, activation=act,
                              max_num_neighbors=1000)
    return model.to(device)


def _config2(args, capturable=False):
    """The config-2 model, its force-matching step function, the AdamW and
    the resident batch (fresh model from the benchmark seed)."""
    import torch

    from mlcg_amd import nn, synthetic

    dev = torch.device("cuda:0")
    torch.manual_seed(synthetic.seed_for(2))
    model = build_model(torch, nn, dev)
    gm = nn.GradientsOut(model).train()
    loss_fn = nn.ForceMSE()
    # torch's fused AdamW: the update in one multi-tensor kernel launch per
    # chunk instead of one per elementwise stage
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, weight_decay=0.0, fused=True,
                            capturable=capturable)
    data = synthetic.config2(n_frames=args.frames).to_torch(dev)

    def step(d=data):
        opt.zero_grad(set_to_none=True)
        out = gm(d)
        out.out.update(**out.out[model.name])
        loss = loss_fn(out)
        loss.backward()
        opt.step()
        return loss

    return model, step, opt, data


def _device_ms_per_step(step, k=5):
    """Device time of k steps with the host issue kept off the critical
    path: a spin kernel holds the stream while the host queues the k steps,
    and HIP events bracket the steps behind it."""
    import torch

    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    torch.cuda._sleep(1_000_000)
    e1.record()
    torch.cuda.synchronize()
    cyc_per_ms = 1_000_000 / max(e0.elapsed_time(e1), 1e-3)
    # enough spin for the host to queue every step (generously: 10 ms each)
    torch.cuda._sleep(int(cyc_per_ms * 10.0 * k))
    e0.record()
    for _ in range(k):
        step()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / k


def _host_issue_ms(step, reps=7):
    """Host time for step() to return (no synchronisation inside), each
    repetition starting from an idle, drained stream."""
    import torch

    t = []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        step()
        t.append((time.perf_counter() - t0) * 1e3)
    torch.cuda.synchronize()
    return statistics.median(t)


def _timed_steps(step, steps):
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps, loss


def gpu_leg(args):
    import torch

    from mlcg_amd import _lib
    from mlcg_amd.nn import _fused

    model, step, opt, data = _config2(args)
    graph = model.build_graph(data)
    E, P, N, B = graph.num_edges, graph.num_pairs, graph.num_nodes, int(data.n_atoms.numel())
    del graph
    if not args.exact_graph:
        # fixed-capacity radius graph: no host synchronisation inside the step
        # (the edge count stays on the device); overflow is checked after the
        # timed region, so the graph used is exactly the one sized above
        cap = int(E * 1.02) + 64
        model.graph_capacity = cap + (cap % 2)

    for _ in range(max(args.warmup, 1)):
        step()
    torch.cuda.synchronize()
    # per-kernel profiling pass (outside the timed region), every HIP entry
    # point bracketed by events, with the whole step on one stream (filter
    # forwards in block order, weight-gradient reductions inline) so that no
    # launch shares the GPU with another stream's work: stand-alone times
    ahead, side = _fused._FILTER_AHEAD, _fused._TMM_SIDE
    _fused._FILTER_AHEAD = _fused._TMM_SIDE = False
    n_prof = 3
    timer = _lib.LaunchTimer(None)
    _lib.set_timer(timer)
    for _ in range(n_prof):
        step()
    torch.cuda.synchronize()
    _lib.set_timer(None)
    _fused._FILTER_AHEAD, _fused._TMM_SIDE = ahead, side
    warm = kernel_report(timer.summary(), E, P, N, B, timer.work())
    per_step = {k: v["total_ms"] / n_prof for k, v in warm.items()}
    dominant = max(per_step, key=per_step.get)

    # timed region: only the dominant kernel's launches are bracketed (HIP
    # events on the stream it runs on)
    timer = _lib.LaunchTimer({dominant})
    _lib.set_timer(timer)
    ms, loss = _timed_steps(step, args.steps)
    _lib.set_timer(None)
    assert math.isfinite(float(loss.detach())), "non-finite loss"
    if model.graph_capacity is not None:
        flags = int(model.last_graph.flags.item())
        assert flags == 0, f"radius graph overflowed its capacity (flags {flags})"
        assert int(model.last_graph.rowptr[-1]) == E, "edge count changed"
    dom = kernel_report(timer.summary(), E, P, N, B, timer.work())[dominant]
    # where the eager step's time goes: the host's issue time of one step
    # and the device time of a step queued ahead of the GPU
    host_ms = _host_issue_ms(step)
    dev_ms = _device_ms_per_step(step)
    # the same step with the filter forwards in block order on one stream
    _fused._FILTER_AHEAD = False
    step()
    noahead_ms, _ = _timed_steps(step, args.steps)
    noahead_dev_ms = _device_ms_per_step(step)
    _fused._FILTER_AHEAD = ahead
    # the same step with the filter forward on the fp32 MFMA throughout
    # (MLCG_FILTER_FP32_STRICT) instead of split-fp16 products, for comparison
    model.strict_fp32_filters = True
    for _ in range(2):
        step()
    strict_ms, _ = _timed_steps(step, args.steps)
    model.strict_fp32_filters = False
    return {"ms_per_step": ms, "E": E, "P": P, "N": N, "B": B, "dominant": dominant,
            "strict_fp32_ms_per_step": strict_ms,
            "host_issue_ms": host_ms, "device_ms": dev_ms,
            "filter_ahead_off": {"ms_per_step": round(noahead_ms, 4),
                                 "device_ms_per_step": round(noahead_dev_ms, 4)},
            "dominant_row": dom, "kernels": warm, "loss": float(loss.detach()),
            "step_kernel_ms": round(sum(per_step.values()), 4)}


def captured_leg(args, E):
    """The same config-2 training step recorded once as a HIP graph
    (mlcg_amd.pl.CapturedTrainStep: capturable AdamW, warm-up and capture on
    a side stream) and replayed: one host launch per step.  Every timed step
    first loads its batch into the recorded inputs (device-to-device copies
    of positions, forces, types, batch vector and frame sizes from a second
    resident copy of the batch), as a training loop feeding new batches
    would.  Fresh model and optimizer from the same seed as the eager leg."""
    import torch

    from mlcg_amd.pl import CapturedTrainStep

    model, step, opt, data = _config2(args, capturable=True)
    cap = int(E * 1.02) + 64
    model.graph_capacity = cap + (cap % 2)
    cs = CapturedTrainStep(lambda d: step(d), data, model, opt, warmup=3)
    batch = data.clone()

    def replay():
        return cs.step(batch)

    for _ in range(max(args.warmup, 1)):
        replay()
    ms, loss = _timed_steps(replay, args.steps)
    dev_ms = _device_ms_per_step(replay)
    loss = float(loss.detach())
    assert math.isfinite(loss), "non-finite loss in the captured step"
    cs.check()
    assert int(model.last_graph.rowptr[-1]) == E, "edge count changed"
    return {"ms_per_step": ms, "device_ms_per_step": round(dev_ms, 4),
            "edges_per_s": E * N_BLOCKS / (ms * 1e-3), "loss": loss}


def gather_ceiling_leg(reps=10):
    """What the CFConv gather kernel (mlcg_cfconv_gather: one wave per
    receiver row, each half-wave reading one 512-byte filter row and one node
    row per edge as float4 lanes) reaches on synthetic CSR graphs whose
    access pattern is controlled, all with the caches flushed (a 1 GiB read)
    before every timed launch, beside torch's streaming reads of the same
    filter bytes:
      config2     the config-2 radius graph (each pair's filter row read from
                  both of its rows, node rows of the frame); also after a
                  1 GiB write (dirty caches, as in the training step)
      seq_unique  24 edges per row, every edge its own filter row, rows in
                  address order, node row = the receiver's own (cached)
      rand_unique the same with the filter rows in a random order
    Bytes are the algorithmic ones (filter rows read once, node rows once,
    output once)."""
    import torch

    from mlcg_amd import ops, synthetic

    dev = torch.device("cuda:0")
    F = 128
    flush = torch.empty(256 * 1024 * 1024, dtype=torch.float32, device=dev)
    gen = torch.Generator(device=dev).manual_seed(7)

    flush.fill_(1.0)
    torch.cuda.synchronize()

    def timed(fn, dirty=False):
        ts = []
        for _ in range(reps):
            # a 1 GiB read evicts the caches and leaves them clean; a 1 GiB
            # write (dirty=True) leaves them full of dirty lines whose write-back
            # competes with the timed reads -- the state after the filter
            # forward, which writes W and W' just before the gathers
            if dirty:
                flush.fill_(1.0)
            else:
                flush.sum()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e-3)
        return statistics.median(ts)

    out = {}
    b = synthetic.config2(n_frames=512)
    pos = torch.from_numpy(b.pos).to(dev)
    g = ops.radius_graph(pos, 20.0, torch.from_numpy(b.batch).to(dev), max_num_neighbors=1000,
                         with_pairs=True)
    N, P, E = g.num_nodes, g.num_pairs, g.num_edges
    y = torch.randn(N, F, device=dev, generator=gen)
    W = torch.randn(g.pair_capacity, F, device=dev, generator=gen)
    byt = 4 * F * (P + 2 * N) + 4 * (N + 1) + 8 * E
    for dirty in (False, True):
        t = timed(lambda: ops.cfconv_gather(y, W, g), dirty)
        out["config2" + ("_dirty_caches" if dirty else "")] = {
            "us": round(t * 1e6, 2), "TB_per_s": round(byt / t / 1e12, 3), "bytes": byt,
            "edges": E}
    deg = 24
    Eu = N * deg
    rowptr = torch.arange(0, Eu + 1, deg, dtype=torch.int32, device=dev)
    col = torch.arange(N, dtype=torch.int32, device=dev).repeat_interleave(deg)
    Wu = torch.randn(Eu, F, device=dev, generator=gen)
    for name, e2p in (("seq_unique", torch.arange(Eu, dtype=torch.int32, device=dev)),
                      ("rand_unique", torch.randperm(Eu, generator=gen, device=dev)
                       .to(torch.int32))):
        gu = ops.PairGraph(edge_index=None, rowptr=rowptr, col=col, pair_ij=None, pairptr=None,
                           eid2pair=e2p, frame_ptr=None, num_nodes=N, num_edges=Eu,
                           num_pairs=Eu)
        t = timed(lambda: ops.cfconv_gather(y, Wu, gu))
        byt = 4 * F * (Eu + 2 * N) + 4 * (N + 1) + 8 * Eu
        out[name] = {"us": round(t * 1e6, 2), "TB_per_s": round(byt / t / 1e12, 3),
                     "bytes": byt, "edges": Eu}
    t = timed(lambda: Wu.sum(dtype=torch.float32))
    out["torch_sum_same_bytes"] = {"us": round(t * 1e6, 2),
                                   "TB_per_s": round(4 * F * Eu / t / 1e12, 3)}
    dst = torch.empty_like(Wu)
    t = timed(lambda: dst.copy_(Wu))
    out["torch_copy_same_bytes"] = {"us": round(t * 1e6, 2),
                                    "TB_per_s_read_plus_write": round(8 * F * Eu / t / 1e12, 3)}
    del flush
    return out


def stream_leg(reps=5):
    """The HBM ceiling of this part, measured with this library's streaming
    kernels (mlcg_stream_read / mlcg_stream_copy: grid-stride loops, 16-byte
    loads, `unroll` loads in flight per thread), caches evicted by a 1 GiB
    read before every timed launch.  Sizes: 1 GiB (the asymptote) and the
    byte counts of the config-2 gathers (~130 and ~250 MB) and of one node
    tensor (9 MB), where launch ramp-up and tail are part of the time.  For
    every size the best launch shape of the sweep is kept."""
    import torch

    from mlcg_amd import _lib

    dev = torch.device("cuda:0")
    flush = torch.ones(256 * 1024 * 1024, dtype=torch.float32, device=dev)
    partial = torch.empty(65536, dtype=torch.float32, device=dev)
    sizes = {"1GiB": 1 << 30, "250MB": 250_000_000, "130MB": 130_000_000, "9MB": 9_175_040}
    src = torch.ones((1 << 30) // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = {}
    for label, nbytes in sizes.items():
        n = (nbytes // 16) * 4
        best = {}
        for kind in ("read", "copy"):
            for groups in (512, 1024, 2048, 4096, 8192):
                for unroll in (4, 8, 16):
                    ts = []
                    for _ in range(reps):
                        flush.sum()
                        torch.cuda.synchronize()
                        e0 = torch.cuda.Event(enable_timing=True)
                        e1 = torch.cuda.Event(enable_timing=True)
                        e0.record()
                        if kind == "read":
                            _lib.call("mlcg_stream_read", src.data_ptr(), n, groups, unroll,
                                      partial.data_ptr(), stream)
                        else:
                            _lib.call("mlcg_stream_copy", src.data_ptr(), dst.data_ptr(), n,
                                      groups, unroll, stream)
                        e1.record()
                        torch.cuda.synchronize()
                        ts.append(e0.elapsed_time(e1) * 1e-3)
                    t = statistics.median(ts)
                    moved = 4 * n * (1 if kind == "read" else 2)
                    gbs = moved / t / 1e9
                    if kind not in best or gbs > best[kind]["GB_per_s"]:
                        best[kind] = {"GB_per_s": round(gbs, 1), "us": round(t * 1e6, 2),
                                      "groups": groups, "unroll": unroll,
                                      "frac_of_8TBs": round(gbs / HBM_PEAK_GBS, 4)}
        out[label] = best
    del flush, src, dst
    return out


MFMA_PEAKS = {  # published dense peaks of the part (TFLOP/s)
    "f16_16x16x32": 2500.0, "f16_16x16x16": 2500.0, "f32_16x16x4": 157.3,
    "bf16_16x16x32": 2500.0, "f16_32x32x16": 2500.0}


def mfma_leg(reps=5):
    """The sustained matrix-core rate of this part for each MFMA shape the
    kernels use (mlcg_mfma_loop: 8 independent accumulator chains per wave on
    register operands), for 1 to 4 workgroups of 4 waves per CU; the best
    median of `reps` launches is kept per shape."""
    import torch

    from mlcg_amd import _lib

    dev = torch.device("cuda:0")
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    out = {}
    for kind, label in enumerate(MFMA_PEAKS):
        fpw = int(lib.mlcg_mfma_loop_flops_per_wave_iter(kind))
        best = None
        for per_cu in (1, 2, 4):
            groups = n_cu * per_cu
            buf = torch.empty(groups * 256, dtype=torch.float32, device=dev)
            iters = 4096 if kind != 2 else 1024
            _lib.call("mlcg_mfma_loop", kind, iters, groups, buf.data_ptr(), stream)
            ts = []
            for _ in range(reps):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                _lib.call("mlcg_mfma_loop", kind, iters, groups, buf.data_ptr(), stream)
                e1.record()
                torch.cuda.synchronize()
                ts.append(e0.elapsed_time(e1) * 1e-3)
            assert bool(torch.isfinite(buf).all())
            t = statistics.median(ts)
            tf = groups * 4 * iters * fpw / t / 1e12
            if best is None or tf > best["TFLOP_per_s"]:
                best = {"TFLOP_per_s": round(tf, 1), "us": round(t * 1e6, 1),
                        "groups_per_cu": per_cu, "iters": iters,
                        "frac_of_peak": round(tf / MFMA_PEAKS[label], 4)}
        out[label] = best
    return out


def radius_leg(reps=10):
    """Config 3 radius graph, inputs resident in HBM.  Figures: the exactly
    sized call end to end (sizing pass, one host synchronisation to size the
    output as the reference's radius.cu:288, write pass), the fixed-capacity
    call (one launch, no synchronisation: the form a captured step uses),
    and the device time of each entry point (HIP events around the call);
    the roofline takes the fixed-capacity form's."""
    import torch

    from mlcg_amd import _lib, ops, synthetic

    b = synthetic.config3()
    pos = torch.from_numpy(b.pos).cuda()
    batch = torch.from_numpy(b.batch).cuda()
    nf = b.n_frames
    fptr = ops.frame_ptr_from_batch(batch, nf)
    for _ in range(2):
        g = ops.radius_graph(pos, 15.0, batch, False, 1000, frame_ptr=fptr)
    torch.cuda.synchronize()
    E = g.num_edges
    cap = E + 1024

    def timed(fn):
        t = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            t.append(time.perf_counter() - t0)
        return statistics.median(t)

    s_exact = timed(lambda: ops.radius_graph(pos, 15.0, batch, False, 1000, frame_ptr=fptr))
    gc = ops.radius_graph(pos, 15.0, batch, False, 1000, frame_ptr=fptr, capacity=cap)
    s_cap = timed(lambda: ops.radius_graph(pos, 15.0, batch, False, 1000, frame_ptr=fptr,
                                           capacity=cap))
    gc = ops.radius_graph(pos, 15.0, batch, False, 1000, frame_ptr=fptr, capacity=cap)
    torch.cuda.synchronize()
    assert int(gc.flags.item()) == 0 and int(gc.rowptr[-1].item()) == E

    def device_ms(names, **kw):
        timer = _lib.LaunchTimer(set(names))
        _lib.set_timer(timer)
        for _ in range(reps):
            ops.radius_graph(pos, 15.0, batch, False, 1000, frame_ptr=fptr, **kw)
        torch.cuda.synchronize()
        _lib.set_timer(None)
        summ = timer.summary()
        return {k: summ[k][1] / summ[k][0] for k in names}

    fused = device_ms(("mlcg_radius_graph",), capacity=cap)
    exact = device_ms(("mlcg_radius_rowptr", "mlcg_radius_fill"))
    dev_ms = fused["mlcg_radius_graph"]
    nbytes = 12 * pos.shape[0] + 8 * (nf + 1) + 16 * E
    ach = nbytes / (dev_ms * 1e-3) / 1e9
    return {"workload": "config3: 2048 frames x 100-bead globules, rc 15 A, no loops, "
                        "int64 [2,E] canonical order",
            "E": E, "ms": round(s_exact * 1e3, 4), "edges_per_s": E / s_exact,
            "ms_capacity_form": round(s_cap * 1e3, 4), "edges_per_s_capacity_form": E / s_cap,
            "kernels_device_ms": round(dev_ms, 4),
            "kernels_avg_us": {k: round(v * 1e3, 2) for k, v in {**fused, **exact}.items()},
            "exact_form_device_ms": round(sum(exact.values()), 4),
            "algorithmic_bytes": nbytes,
            "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                         "time": "device time of mlcg_radius_graph (one launch: sweep, "
                                 "look-back and write)"}}


def fp16_leg(reps=5):
    """Config 4: 256 frames x 500-bead globules, rc 15 A, fp16 filter linears
    with fp32 accumulation; energy + forces (inference) per call."""
    import torch

    from mlcg_amd import _lib, nn, synthetic

    dev = torch.device("cuda:0")
    torch.manual_seed(synthetic.seed_for(4))
    rbf = nn.GaussianBasis(nn.CosineCutoff(0.0, 15.0), num_rbf=K_RBF)
    model = nn.StandardSchNet(rbf, nn.CosineCutoff(0.0, 15.0), [64], H, 100, F, N_BLOCKS,
                              torch.nn.Tanh()).to(dev)
    model.fp16_filters = True
    gm = nn.GradientsOut(model).eval()
    b = synthetic.config4()
    data = b.to_torch(dev)
    from mlcg_amd.nn import _fused

    with torch.no_grad():
        gm(data)
        torch.cuda.synchronize()
        E, P = model.last_graph.num_edges, model.last_graph.num_pairs
        t = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            gm(data)
            torch.cuda.synchronize()
            t.append(time.perf_counter() - t0)
        # the filter kernel's stand-alone launch time: filter forwards in
        # block order on one stream, bracketed by events
        ahead = _fused._FILTER_AHEAD
        _fused._FILTER_AHEAD = False
        timer = _lib.LaunchTimer({"mlcg_filter_fwd"})
        _lib.set_timer(timer)
        for _ in range(2):
            gm(data)
        torch.cuda.synchronize()
        _lib.set_timer(None)
        _fused._FILTER_AHEAD = ahead
    s = statistics.median(t)
    n_l, tot = timer.summary()["mlcg_filter_fwd"]
    avg = tot / n_l
    flops = 2 * 2 * (K_RBF * F + F * F) * P
    ach = flops / (avg * 1e-3) / 1e12
    return {"workload": "config4: 256 frames x 500-bead globules, rc 15 A, fp16 filter "
                        "linears (fp32 accumulate), energy + forces",
            "edges": E, "ms_per_call": round(s * 1e3, 3),
            "cfconv_edges_per_s": E * N_BLOCKS / s, "frames_per_s": b.n_frames / s,
            "filter_roofline": {"kernel": "filter_fwd_f16_kernel", "bound": "mfma",
                                "achieved": round(ach, 2), "peak": FP16_MFMA_PEAK_TFLOPS,
                                "unit": "TFLOP/s", "frac": round(ach / FP16_MFMA_PEAK_TFLOPS, 4),
                                "avg_launch_us": round(avg * 1e3, 2)}}


def md_leg(steps):
    """Config 5: 100 replicas x 268-bead chains, config-2 SchNet (rc 20 A) +
    bonds, angles, 3-term dihedrals and (sigma/r)^6 repulsion, BAOAB at 300 K,
    dt 4 fs, friction 1/ps; radius graph rebuilt every step; the step is
    captured once as a HIP graph and replayed.  The per-kernel report comes
    from a few eager force evaluations on the final state (HIP events cannot
    bracket launches inside a replayed graph)."""
    import torch

    from mlcg_amd import _lib, nn, synthetic
    from mlcg_amd.simulation import LangevinSimulation

    c = synthetic.CONFIG5_PRIORS
    torch.manual_seed(synthetic.seed_for(5))
    rbf = nn.GaussianBasis(nn.CosineCutoff(0.0, RC), num_rbf=K_RBF)
    schnet = nn.StandardSchNet(rbf, nn.CosineCutoff(0.0, RC), [64], H, 100, F, N_BLOCKS,
                               torch.nn.Tanh())
    models = {"SchNet": nn.GradientsOut(schnet)}
    for k, v in synthetic.config5_prior_models().items():
        models[k] = nn.GradientsOut(v)
    model = nn.SumOut(torch.nn.ModuleDict(models))
    confs = synthetic.config5_configurations()
    beta = 1.0 / (0.0019872041 * c["temperature_K"])
    # an untimed warm-up run first (the first simulation of a process runs
    # 5-20 % slower: clocks, first-touch of the graph's memory), then the
    # timed one from the same configurations
    for n in (53, steps + 3):
        sim = LangevinSimulation(friction=c["friction_per_ps"], dt=c["dt_ps"], n_timesteps=n,
                                 save_interval=n, random_seed=synthetic.seed_for(5),
                                 capture=True, check_interval=n)
        sim.attach_model_and_configurations(model, confs, beta)
        sim.simulate()
    sps = sim.timed_steps / sim.timed_seconds
    # per-kernel device times of the force evaluation, eagerly, on the final state
    from mlcg_amd.nn import _fused

    data = sim.final_data
    ahead = _fused._FILTER_AHEAD
    _fused._FILTER_AHEAD = False  # one stream: stand-alone launch times
    with torch.no_grad():
        model(data)
        torch.cuda.synchronize()
        timer = _lib.LaunchTimer(None)
        _lib.set_timer(timer)
        reps = 3
        for _ in range(reps):
            model(data)
        torch.cuda.synchronize()
        _lib.set_timer(None)
    _fused._FILTER_AHEAD = ahead
    g = schnet.last_graph
    N = data.pos.shape[0]
    E = int(g.rowptr[-1].item())
    P = int(g.pairptr[-1].item())
    summ = {k: (v[0] // reps, v[1] / reps) for k, v in timer.summary().items()}
    rows = kernel_report(summ, E, P, N, sim.n_sims,
                         {k: v / reps for k, v in timer.work().items()})
    dom = max(rows, key=lambda k: rows[k]["total_ms"])
    d = rows[dom]
    roof = {k: d.get(k) for k in ("bound", "achieved", "peak", "unit", "frac")}
    roof.update(kernel=d["kernel"], avg_launch_us=d["avg_us"], launches_per_step=d["launches"])
    return {"workload": "config5: 100 x 268-bead chains, SchNet (3 blocks, rc 20 A) + "
                        "bonds/angles/dihedrals/repulsion priors, BAOAB, HIP-graph step",
            "steps_timed": sim.timed_steps, "ms_per_step": round(1e3 / sps, 4),
            "steps_per_s": sps, "replica_steps_per_s": sps * sim.n_sims,
            "edges": E, "pairs": P, "edge_capacity": schnet.graph_capacity,
            "roofline": roof,
            "kernels": {k: {kk: v[kk] for kk in ("kernel", "launches", "avg_us", "frac")
                            if kk in v} for k, v in rows.items()},
            "prior_constants": c}


def cpu_model() -> str:
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, warmups=2, reps=5):
    for _ in range(warmups):
        fn()
    t = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        t.append(time.perf_counter() - t0)
    return statistics.median(t), len(t)


def cpu_leg(args):
    """The CPU restatement (oracle/, this repository's op-by-op restatement of
    the reference, run in fp32) of the config-2 step on a bounded sample of
    frames: 2 warm-ups, then the median of at least 5 runs."""
    import torch

    from mlcg_amd import synthetic
    from oracle import radius as oracle_radius
    from oracle import schnet_ref as R

    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    torch.set_float32_matmul_precision("highest")
    cfg = R.SchNetConfig(num_rbf=K_RBF, rbf_lo=0.0, rbf_hi=RC, rbf_cut="cosine",
                         conv_cut="cosine", conv_lo=0.0, conv_hi=RC, act="tanh",
                         num_blocks=N_BLOCKS)
    sd = R.random_state_dict(cfg, seed=synthetic.seed_for(2))
    b = synthetic.config2(n_frames=args.cpu_frames)
    pos = torch.from_numpy(b.pos)
    types = torch.from_numpy(b.atom_types)
    batch = torch.from_numpy(b.batch)
    fref = torch.from_numpy(b.forces)

    def one():
        ei, _ = oracle_radius.radius_graph(b.pos, RC, b.batch, False, 1000)
        ei = torch.from_numpy(ei)
        R.force_matching_grads(sd, cfg, pos, types, batch, ei, b.n_frames, fref)
        return ei.shape[1]

    E = one()  # warm-up
    t = []
    t_start = time.perf_counter()
    while len(t) < 5 or (time.perf_counter() - t_start < args.cpu_seconds and len(t) < 50):
        t0 = time.perf_counter()
        one()
        t.append(time.perf_counter() - t0)
    s = statistics.median(t)
    return {"value": E * N_BLOCKS / s, "unit": "edges/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{args.cpu_frames} frames of the config-2 workload (E={E}), "
                      f"oracle/schnet_ref.py fp32 force-matching step incl. brute-force "
                      f"radius graph, median of {len(t)} reps, torch threads={cores}",
            "ms_per_step": round(s * 1e3, 3)}


def cpu_configs_leg():
    """CPU baselines of configs 1, 3, 4 and 5 (the reference's own CPU-runnable
    case, the radius-graph, fp16 and MD configurations): the
    oracle restatements in fp32 on the host cores, 2 warm-ups then the median
    of 5 (configs 1, 3, 4), and 20 steps reported per step (config 5).
    Configs 4 and 5 run on bounded samples (stated in each record)."""
    import math as _m

    import numpy as np
    import torch

    from mlcg_amd import synthetic
    from oracle import langevin_ref as L
    from oracle import priors_ref as P
    from oracle import radius as oracle_radius
    from oracle import schnet_ref as R

    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    torch.set_float32_matmul_precision("highest")
    out = {"cores": cores, "cpu_model": cpu_model(), "kind": "port"}

    def nl(bt, rc):
        ei, _ = oracle_radius.radius_graph(bt.pos, rc, bt.batch, False, 1000)
        return torch.from_numpy(ei)

    def schnet_cfg(blocks, rc, act):
        return R.SchNetConfig(num_rbf=K_RBF, rbf_lo=0.0, rbf_hi=rc, rbf_cut="cosine",
                              conv_cut="cosine", conv_lo=0.0, conv_hi=rc, act=act,
                              num_blocks=blocks)

    # config 1: 1 block, SSP, rc 30, 32 x 10 beads, energy + forces (whole config)
    b1 = synthetic.config1()
    c1 = schnet_cfg(1, 30.0, "ssp")
    sd1 = R.random_state_dict(c1, seed=synthetic.seed_for(1))
    t1 = [torch.from_numpy(x) for x in (b1.pos, b1.atom_types, b1.batch)]
    s, n = _median_time(lambda: R.schnet_energy_forces(sd1, c1, t1[0], t1[1], t1[2],
                                                       nl(b1, 30.0), b1.n_frames))
    E1 = nl(b1, 30.0).shape[1]
    out["config1"] = {"value": E1 / s, "unit": "CFConv edges/s (1 block)",
                      "ms_per_call": round(s * 1e3, 3), "reps": n,
                      "sample": "whole config 1 (32 x 10 beads), energy + forces incl. "
                                "the brute-force radius graph"}
    # config 3: radius graph, whole config, the C brute force (one thread)
    b3 = synthetic.config3()
    s, n = _median_time(lambda: oracle_radius.radius_graph(b3.pos, 15.0, b3.batch, False, 1000))
    E3 = oracle_radius.radius_graph(b3.pos, 15.0, b3.batch, False, 1000)[0].shape[1]
    out["config3"] = {"value": E3 / s, "unit": "radius-graph edges/s",
                      "ms_per_call": round(s * 1e3, 3), "reps": n, "threads": 1,
                      "sample": "whole config 3 (2048 x 100 beads); oracle/radius_ref.c per-frame "
                                "brute force standing in for torch_cluster's kd-tree"}
    # config 4: fp32 energy + forces (the reference's fp32 path; the fp16
    # filter variant is a GPU option) on 8 of the 500-bead globules
    b4 = synthetic.config4(n_frames=8)
    c4 = schnet_cfg(N_BLOCKS, 15.0, "tanh")
    sd4 = R.random_state_dict(c4, seed=synthetic.seed_for(4))
    t4 = [torch.from_numpy(x) for x in (b4.pos, b4.atom_types, b4.batch)]
    ei4 = nl(b4, 15.0)
    s, n = _median_time(lambda: R.schnet_energy_forces(sd4, c4, t4[0], t4[1], t4[2], nl(b4, 15.0),
                                                       b4.n_frames), warmups=1)
    out["config4"] = {"value": ei4.shape[1] * N_BLOCKS / s, "unit": "CFConv edges/s",
                      "ms_per_call": round(s * 1e3, 3), "reps": n,
                      "sample": f"8 of the 256 frames (E={ei4.shape[1]}), fp32 energy + "
                                "forces incl. the radius graph"}
    # config 5: the composite BAOAB step on 2 of the 100 replicas, 20 steps
    c = synthetic.CONFIG5_PRIORS
    nrep, nb = 2, 268
    b5 = synthetic.config5(n_frames=nrep, n_beads=nb)
    c5 = schnet_cfg(N_BLOCKS, RC, "tanh")
    sd5 = R.random_state_dict(c5, seed=synthetic.seed_for(5))
    topo = P.chain_topology(nrep, nb, min_sep=c["repulsion"]["min_separation"])

    def full(M, v):
        return torch.full((M,), float(v))

    prm = {"bonds": {"x0": full(topo["bonds"][0].shape[1], c["bonds"]["x_0"]),
                     "k": full(topo["bonds"][0].shape[1], c["bonds"]["k"])},
           "angles": {"x0": full(topo["angles"][0].shape[1],
                                 _m.cos(_m.radians(c["angles"]["theta_0_deg"]))),
                      "k": full(topo["angles"][0].shape[1], c["angles"]["k"])},
           "dihedrals": {"v_0": full(topo["dihedrals"][0].shape[1], c["dihedrals"]["v_0"]),
                         "k1s": torch.tensor(c["dihedrals"]["k1s"]).repeat(
                             topo["dihedrals"][0].shape[1], 1),
                         "k2s": torch.tensor(c["dihedrals"]["k2s"]).repeat(
                             topo["dihedrals"][0].shape[1], 1)},
           "repulsion": {"sigma": full(topo["repulsion"][0].shape[1], c["repulsion"]["sigma"])}}
    types5 = torch.from_numpy(b5.atom_types)
    batch5 = torch.from_numpy(b5.batch)
    m = torch.full((nrep * nb,), c["masses_amu"] / 418.4)
    beta = 1.0 / (L.KB_KCAL * c["temperature_K"])
    bmr = torch.sqrt(1.0 / (beta * m))
    vs, ns = L.constants(c["dt_ps"], c["friction_per_ps"])
    gen = torch.Generator().manual_seed(5)

    def forces(x):
        ei = torch.from_numpy(oracle_radius.radius_graph(
            x.numpy(), RC, b5.batch, False, 1000)[0])
        _, F = R.schnet_energy_forces(sd5, c5, x, types5, batch5, ei, nrep)
        for kind, (mp, mb) in topo.items():
            F = F + P.prior_energy_forces(kind, x, mp, mb, nrep, prm[kind])[1]
        return F

    x = torch.from_numpy(b5.pos).clone()
    v = torch.randn(x.shape, generator=gen) * bmr[:, None]
    F = forces(x)
    n_steps = 20
    t0 = time.perf_counter()
    for _ in range(n_steps):
        xi = torch.randn(x.shape, generator=gen)
        x, v = L.baoa(x, v, F, m, bmr, c["dt_ps"], vs, ns, xi)
        F = forces(x)
        v = L.b(v, F, m, c["dt_ps"])
    s5 = (time.perf_counter() - t0) / n_steps
    assert bool(np.isfinite(x.numpy()).all())
    out["config5"] = {"value": nrep / s5, "unit": "replica-steps/s",
                      "ms_per_step": round(s5 * 1e3, 3),
                      "ms_per_1000_steps_100_replicas_extrapolated":
                          round(s5 * 1e3 * 1000 * 100 / nrep, 1),
                      "sample": f"{nrep} of the 100 replicas x {nb} beads, {n_steps} BAOAB "
                                "steps, fp32 SchNet + 4 priors + radius graph each step"}
    return out


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): this build has no "
              "multi-GPU path (frames would shard across GPUs with no exchange; only the "
              "parameter-gradient all-reduce of a training step would cross GPUs)",
              file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    if args.calib_copy_mib > 0:
        n = args.calib_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only_probes:
        res = {}
        if args.stream_probe:
            res["stream"] = stream_leg()
        if args.gather_probe:
            res["gather_ceiling"] = gather_ceiling_leg()
        if args.mfma_probe:
            res["mfma"] = mfma_leg()
        print(json.dumps(res))
        return 0
    if args.captured_only:
        model, _, _, data = _config2(args)
        E = model.build_graph(data).num_edges
        del model, data
        cg = captured_leg(args, E)
        print(json.dumps({"captured_step": cg, "E": E}))
        return 0
    sp = stream_leg() if args.stream_probe else None
    if sp:
        print("[bench] stream probe " + json.dumps(sp), flush=True)
    g = gpu_leg(args)
    print(f"[bench] eager leg done: {g['ms_per_step']:.3f} ms/step, E={g['E']}", flush=True)
    cg = None if args.no_capture else captured_leg(args, g["E"])
    if cg:
        print(f"[bench] captured leg done: {cg['ms_per_step']:.3f} ms/step", flush=True)
    gc = gather_ceiling_leg() if args.gather_probe else None
    if gc:
        print(f"[bench] gather probe done: {gc}", flush=True)
    rg = None if args.no_radius else radius_leg()
    if rg:
        print(f"[bench] radius leg done: {rg['ms']:.3f} ms", flush=True)
    f16 = None if args.no_fp16 else fp16_leg()
    if f16:
        print(f"[bench] fp16 leg done: {f16['ms_per_call']:.3f} ms/call", flush=True)
    md = None if args.no_md else md_leg(args.md_steps)
    if md:
        print(f"[bench] md leg done: {md['ms_per_step']:.3f} ms/step", flush=True)
    cpu = None if args.no_cpu else cpu_leg(args)
    if cpu:
        print(f"[bench] cpu leg done: {cpu['ms_per_step']:.1f} ms/step", flush=True)
    cpu_cfg = None if args.no_cpu else cpu_configs_leg()
    if cpu_cfg:
        print("[bench] cpu configs 1, 3, 4, 5 done", flush=True)

    # per-kernel tables go on their own lines before the result line, which
    # stays short enough to be kept whole by a log tail
    print("[bench] config2 kernels " + json.dumps(g["kernels"]), flush=True)
    if md:
        print("[bench] config5 kernels " + json.dumps(md.pop("kernels")), flush=True)
        md.pop("prior_constants", None)
    if cpu_cfg:
        print("[bench] cpu baselines of configs 1, 3, 4, 5 " + json.dumps(cpu_cfg), flush=True)

    # the headline: the training step through mlcg_amd.pl.CapturedTrainStep
    # (one graph launch per step, its batch loaded by one mlcg_copy_batch),
    # whose time does not depend on the host's speed; the eager step (the same
    # kernels launched one by one from Python) is reported beside it
    eager_ms = g["ms_per_step"]
    ms = cg["ms_per_step"] if cg else eager_ms
    value = g["E"] * N_BLOCKS / (ms * 1e-3)
    dom = g["dominant_row"]
    sym = dom["kernel"]
    roofline = {"bound": dom.get("bound"), "achieved": dom.get("achieved"),
                "peak": dom.get("peak"), "unit": dom.get("unit"), "frac": dom.get("frac"),
                "traffic": load_traffic(sym), "kernel": sym,
                "avg_launch_us": dom["avg_us"], "launches": dom["launches"],
                "timed_in": "eager timed region (HIP events around each launch; a graph "
                            "replay cannot bracket its kernels)"}
    kr = g["kernels"]
    brief = {k: {kk: v[kk] for kk in ("avg_us", "frac") if kk in v}
             for k, v in kr.items() if v["total_ms"] / 3 > 0.02}
    line = {
        "metric": "CFConv fwd+force+double-bwd edges/s",
        "value": value,
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded self-avoiding CG chains, random-init weights)",
        "config": {"workload": "config2: SchNet force-matching step (radius graph, energy, "
                               "forces, double backward, AdamW), 512 frames x 35 beads, "
                               "H=F=128, 3 blocks, 50 RBF, rc 20 A",
                   "frames": g["B"], "beads_per_frame": g["N"] // max(g["B"], 1),
                   "edges": g["E"], "pairs": g["P"], "blocks": N_BLOCKS},
        "frames_per_s": g["B"] / (ms * 1e-3),
        "step": ("captured: CapturedTrainStep replay, batch loaded each step" if cg
                 else "eager"),
        "captured_step": ({"device_ms_per_step": cg["device_ms_per_step"], "loss": cg["loss"]}
                          if cg else None),
        "eager_step": {"ms_per_step": round(eager_ms, 4),
                       "edges_per_s": g["E"] * N_BLOCKS / (eager_ms * 1e-3),
                       "host_issue_ms": round(g["host_issue_ms"], 4),
                       "device_ms": round(g["device_ms"], 4),
                       "filter_ahead_off": g["filter_ahead_off"]},
        "strict_fp32_filters_eager_step_ms": round(g["strict_fp32_ms_per_step"], 4),
        "roofline": roofline,
        "kernels_us_frac": brief,
        "step_kernel_ms": g["step_kernel_ms"],
        "radius_graph": rg,
        "fp16_config4": f16,
        "md_config5": md,
        "gather_ceiling": gc,
        "stream_ceiling": sp,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
