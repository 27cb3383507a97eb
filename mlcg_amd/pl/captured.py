"""A training step captured once as a HIP graph and replayed.

The reference trains eagerly (mlcg/pl/model.py:113-131 under Lightning's
loop: zero the gradients, training_step, backward, optimizer step).  On this
build that step is ~140 kernel launches plus the Python and torch dispatch
around them, so on a slow host the GPU waits between launches.  For batches
of one fixed shape (the usual CG case: one molecule, a fixed number of frames
per batch) the whole step can be recorded once and replayed with a single
host call per step.  Each replay first copies the new batch into the
recorded input tensors (device to device); the results are those of the
eager step bit for bit (the kernels, their order and their launch shapes are
the same).

Requirements, checked at construction:
- the optimizer is capturable (``torch.optim.AdamW(..., capturable=True)``);
  a non-capturable optimizer raises inside the capture region;
- every SchNet in the model builds its radius graph into a fixed edge
  capacity (no host synchronisation inside the step).  A model without one
  gets ``capacity_factor`` times the example batch's edge count.  A batch
  with more edges than the capacity sets the graph's overflow flag instead of
  growing it: ``check()`` (one host synchronisation) raises if any replay
  since the last check overflowed.
"""

from __future__ import annotations

from typing import Callable, List, Optional

import torch

from .. import ops

def _schnets(module: torch.nn.Module):
    from ..nn.schnet import SchNet

    return [m for m in module.modules() if isinstance(m, SchNet)]


def _tensor_fields(data) -> List[str]:
    return [k for k in data.keys() if isinstance(data[k], torch.Tensor)]


class CapturedTrainStep:
    """``step_fn(data) -> loss`` recorded as one HIP graph.

    step_fn runs one whole training step on ``data`` (zero_grad, forward,
    loss, backward, optimizer.step) and returns the loss tensor.  ``data`` is
    the example batch; its tensors become the graph's inputs, so keep it
    alive.  ``step(batch)`` copies batch's tensors into them (the same keys,
    shapes and dtypes) and replays; it returns the recorded loss tensor,
    overwritten by each replay.

    ``warmup`` eager steps run first on a side stream (torch's capture rules:
    the allocator and lazily built state must exist before recording); they
    update the parameters like any other training step.
    """

    def __init__(self, step_fn: Callable, data, model: torch.nn.Module,
                 optimizer: torch.optim.Optimizer, warmup: int = 3,
                 capacity_factor: float = 1.25):
        if not data.pos.is_cuda:
            raise RuntimeError("CapturedTrainStep needs the batch on a ROCm device")
        for group in optimizer.param_groups:
            if not group.get("capturable", False):
                raise RuntimeError(
                    "CapturedTrainStep needs a capturable optimizer, e.g. "
                    "torch.optim.AdamW(params, ..., capturable=True)")
        self.model = model
        self.data = data
        self.fields = _tensor_fields(data)
        self.schnets = _schnets(model)
        for m in self.schnets:
            if m.graph_capacity is None:
                e = m.build_graph(data).num_edges
                cap = int(e * capacity_factor) + 64
                m.graph_capacity = cap + (cap % 2)
        dev = data.pos.device
        # OR of every replay's radius-graph flags, accumulated on the device
        # inside the graph, so an overflow between two checks is not lost
        self.sticky = torch.zeros(1, dtype=torch.int32, device=dev)

        def recorded(d):
            loss = step_fn(d)
            for m in self.schnets:
                if m.last_graph is not None and m.last_graph.flags is not None:
                    self.sticky.bitwise_or_(m.last_graph.flags)
            return loss

        self._side = torch.cuda.Stream(device=dev)
        self._side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self._side):
            for _ in range(max(int(warmup), 1)):
                recorded(data)
        torch.cuda.current_stream(dev).wait_stream(self._side)
        # the graph's radius-graph workspaces, zero-filled here once rather
        # than by a fill recorded into (and rerun by) every replay
        self._radius_ws = ops.reserve_radius_workspaces(data.pos.shape[0], dev,
                                                        len(self.schnets))
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(self.graph, stream=self._side):
                self.loss = recorded(data)
        finally:
            ops.release_radius_workspaces(dev)
        torch.cuda.synchronize(dev)

    def load(self, batch) -> None:
        """Copy batch's tensors into the recorded inputs (same keys, shapes
        and dtypes), on the current stream, in one launch (ops.copy_batch)
        when they are resident on the recorded device."""
        dsts, srcs = [], []
        for k in self.fields:
            src = batch[k] if k in batch else None
            dst = self.data[k]
            if src is None or src.shape != dst.shape or src.dtype != dst.dtype:
                raise RuntimeError(
                    f"CapturedTrainStep: batch field {k!r} must match the recorded one "
                    f"({tuple(dst.shape)}, {dst.dtype}); got "
                    f"{None if src is None else (tuple(src.shape), src.dtype)}")
            if src.data_ptr() != dst.data_ptr():
                if src.device != dst.device:  # host batches: one upload each
                    src = src.to(dst.device, non_blocking=True)
                src = src.contiguous()
                if (dst.is_contiguous() and dst.data_ptr() % 16 == 0
                        and src.data_ptr() % 16 == 0):
                    dsts.append(dst)
                    srcs.append(src)
                else:  # a strided or unaligned recorded input
                    dst.copy_(src, non_blocking=True)
        if dsts:
            ops.copy_batch(dsts, srcs)

    def step(self, batch=None) -> torch.Tensor:
        """One training step on batch (default: the recorded inputs as they
        are); returns the loss tensor of this replay."""
        if batch is not None:
            self.load(batch)
        self.graph.replay()
        return self.loss

    def check(self) -> None:
        """Raise if the radius graph of any step so far (warm-up steps and
        replays) overflowed its edge capacity or max_num_neighbors, or a
        split-fp16 filter kernel met a value past its range
        (ops.check_numerics); one host synchronisation, the flags are cleared
        afterwards."""
        ops.check_numerics(self.data.pos.device)
        flags = int(self.sticky.item())
        if flags:
            self.sticky.zero_()
            ops.radius_flags_read(flags)
            if flags & 8:  # a look-back timed out: the graph's workspaces restart
                for ws in self._radius_ws:
                    ws.zero_()
            msg = ops.radius_flags_message(flags, [m.graph_capacity for m in self.schnets])
            hint = ("rebuild the CapturedTrainStep with a larger capacity_factor or "
                    "max_num_neighbors" if flags & 3 else
                    "an internal failure of the radius kernel; rebuild the CapturedTrainStep")
            raise RuntimeError(f"radius graph of a captured step reported flags {flags} "
                               f"({msg}): {hint}")
