from .atomic_data import AtomicData, collate
from ._keys import ENERGY_KEY, FORCE_KEY

__all__ = ["AtomicData", "collate", "ENERGY_KEY", "FORCE_KEY"]
