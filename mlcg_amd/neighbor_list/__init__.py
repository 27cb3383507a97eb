from .neighbor_list import (atomic_data2neighbor_list, hip_neighbor_list, make_neighbor_list,
                            validate_neighborlist)
from .radius import radius_distance, radius_graph

__all__ = ["atomic_data2neighbor_list", "hip_neighbor_list", "make_neighbor_list",
           "validate_neighborlist", "radius_distance", "radius_graph"]
