"""Training-step integration (mlcg/pl/model.py) without PyTorch Lightning."""

from .model import PLModel, detect_nan_parameters, train_epoch

__all__ = ["PLModel", "detect_nan_parameters", "train_epoch"]
