"""Training-step integration (mlcg/pl/model.py) without PyTorch Lightning."""

from .captured import CapturedTrainStep
from .model import PLModel, detect_nan_parameters, train_epoch

__all__ = ["CapturedTrainStep", "PLModel", "detect_nan_parameters", "train_epoch"]
