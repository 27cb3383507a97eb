"""The reference's training-step interface, mlcg/pl/model.py:19-131, without
PyTorch Lightning (not part of this build).

`PLModel` keeps the reference's method names and semantics -- step() runs
the model with gradients on for training or for derivative models, merges
the model's outputs into `data.out`, evaluates the loss and returns
(loss, batch size); validation losses of an epoch are combined as the
batch-size weighted mean per metaset (model.py:56-88) -- and stands in for
Lightning's `self.log` by keeping the last logged values in `self.logged`.
`train_epoch` is the loop Lightning's Trainer runs over one epoch (zero the
gradients, training_step, backward, optimizer step), and
`configure_optimizers` builds the AdamW of the reference's training YAMLs
(examples/input_yamls/train_schnet.yaml:92-96).
"""

from __future__ import annotations

from copy import deepcopy
from typing import Dict, Iterable, List, Tuple

import torch

from ..data._keys import N_ATOMS_KEY
from ..nn.gradients import GradientsOut


def detect_nan_parameters(model: torch.nn.Module) -> None:
    """Raise ValueError naming the first parameter with non-finite entries
    (mlcg/utils.py:283-296)."""
    for name, param in model.named_parameters():
        if not torch.isfinite(param).all():
            raise ValueError(f"Detected nan and/or inf values in `{name}`."
                             " Check your forward pass for numerically unstable operations.")


class PLModel(torch.nn.Module):
    """Training interface for the models of `mlcg_amd.nn` (model.py:19-51).

    model: a model whose forward fills `data.out[model.name]` (e.g.
    GradientsOut(SchNet(...))); loss: an `mlcg_amd.nn.Loss`.  Move the
    PLModel to the device (`.to("cuda")`), as Lightning does, so that the
    loss weights live next to the model."""

    def __init__(self, model: torch.nn.Module, loss: torch.nn.Module) -> None:
        super().__init__()
        self.model = model
        self.loss = loss
        self.validation_step_outputs: List[Tuple[torch.Tensor, int]] = []
        self.logged: Dict[str, torch.Tensor] = {}
        self.derivative = getattr(self.model, "derivative", False)
        for module in self.modules():
            if isinstance(module, GradientsOut):
                self.derivative = True

    # -- Lightning hooks ------------------------------------------------
    def log(self, name: str, value, **kwargs) -> None:
        self.logged[name] = value.detach() if torch.is_tensor(value) else value

    def on_train_epoch_start(self) -> None:
        if torch.cuda.is_available():
            torch.cuda.empty_cache()

    def on_train_epoch_end(self) -> None:
        detect_nan_parameters(self.model)
        p = next(self.model.parameters(), None)
        if p is not None and p.is_cuda:
            from .. import ops

            ops.check_numerics(p.device)  # split-fp16 range flags of the epoch

    def on_validation_epoch_end(self) -> torch.Tensor:
        """Mean over batches of the batch-size weighted validation loss per
        metaset (model.py:56-88); logged as `validation_loss`."""
        with torch.no_grad():
            out = torch.tensor([[float(torch.as_tensor(l).detach()), float(b)]
                                for l, b in self.validation_step_outputs],
                               dtype=torch.float64)  # [batches, 2] (or [metasets, batches, 2])
            if out.dim() != 3:
                out = out.view(1, *out.shape)
            out = out[:, :, 0] * out[:, :, 1] / out[:, :, 1].sum(dim=0, keepdim=True)
            out = out.sum(dim=0).mean()
        self.log("validation_loss", out)
        self.validation_step_outputs.clear()
        return out

    # -- steps (model.py:93-131) -----------------------------------------
    def training_step(self, data, batch_idx: int) -> torch.Tensor:
        loss, _ = self.step(data, "train")
        return loss

    def validation_step(self, data, batch_idx: int = 0,
                        dataloader_idx: int = 0) -> Tuple[torch.Tensor, int]:
        loss, batch_size = self.step(data, "validation")
        self.validation_step_outputs.append((loss, batch_size))
        return loss, batch_size

    def test_step(self, data, batch_idx: int = 0,
                  dataloader_idx: int = 0) -> Tuple[torch.Tensor, int]:
        return self.step(data, "test")

    def step(self, data, stage: str) -> Tuple[torch.Tensor, int]:
        with torch.set_grad_enabled(stage == "train" or self.derivative):
            data = self.model(data)
        data.out.update(**data.out[self.model.name])
        loss = self.loss(data)
        batch_size = data[N_ATOMS_KEY].shape[0]
        self.log(f"{stage}_loss", loss)
        return loss, batch_size

    def get_model(self) -> torch.nn.Module:
        return deepcopy(self.model)

    def configure_optimizers(self, lr: float = 1e-4,
                             weight_decay: float = 0.0) -> torch.optim.Optimizer:
        fused = next(self.model.parameters()).is_cuda  # one fused kernel per step on the GPU
        return torch.optim.AdamW(self.model.parameters(), lr=lr, weight_decay=weight_decay,
                                 fused=fused)


def train_epoch(plmodel: PLModel, batches: Iterable, optimizer: torch.optim.Optimizer
                ) -> float:
    """One training epoch as Lightning's loop runs it: per batch, zero the
    gradients, training_step, backward, optimizer step.  Returns the mean
    training loss (a host synchronisation per epoch, none per step)."""
    plmodel.train()
    plmodel.on_train_epoch_start()
    total = None
    n = 0
    for i, data in enumerate(batches):
        optimizer.zero_grad(set_to_none=True)
        loss = plmodel.training_step(data, i)
        loss.backward()
        optimizer.step()
        total = loss.detach() if total is None else total + loss.detach()
        n += 1
    plmodel.on_train_epoch_end()
    return float(total) / max(n, 1) if total is not None else float("nan")
