from .activations import ShiftedSoftplus
from .cutoff import CosineCutoff, IdentityCutoff
from .gradients import EnergyOut, GradientsOut, SumOut
from .losses import EnergyMSE, ForceMSE, ForceRMSE, Loss
from .mlp import MLP, init_xavier_uniform
from .prior import (Dihedral, FourierSeries, Harmonic, HarmonicAngles, HarmonicBonds,
                    Repulsion, StaticDihedral, StaticHarmonicAngles, StaticHarmonicBonds,
                    StaticRepulsion)
from .radial_basis import ExpNormalBasis, GaussianBasis
from .schnet import CFConv, InteractionBlock, SchNet, StandardSchNet

__all__ = ["ShiftedSoftplus", "CosineCutoff", "IdentityCutoff", "EnergyOut", "GradientsOut",
           "SumOut", "EnergyMSE", "ForceMSE", "ForceRMSE", "Loss", "MLP",
           "init_xavier_uniform", "GaussianBasis", "ExpNormalBasis", "CFConv",
           "InteractionBlock", "SchNet", "StandardSchNet", "Harmonic", "HarmonicBonds",
           "HarmonicAngles", "FourierSeries", "Dihedral", "Repulsion", "StaticHarmonicBonds",
           "StaticHarmonicAngles", "StaticDihedral", "StaticRepulsion"]
