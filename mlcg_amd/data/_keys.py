"""Field names of AtomicData (same strings as mlcg/data/_keys.py:14-55)."""

POSITIONS_KEY = "pos"
N_ATOMS_KEY = "n_atoms"
MASS_KEY = "masses"
NEIGHBOR_LIST_KEY = "neighbor_list"
TAG_KEY = "tag"
DIRECTION_VECTORS_KEY = "direction_vectors"
DISTANCES_KEY = "distances"
EDGE_ATTRS_KEY = "edge_attrs"
EDGE_EMBEDDING_KEY = "edge_embedding"
CELL_KEY = "cell"
PBC_KEY = "pbc"
NODE_FEATURES_KEY = "node_features"
NODE_ATTRS_KEY = "node_attrs"
ATOM_TYPE_KEY = "atom_types"
ENERGY_KEY = "energy"
FORCE_KEY = "forces"
VELOCITY_KEY = "velocities"
BATCH_KEY = "batch"

PROPERTY_KEYS = (ENERGY_KEY, FORCE_KEY)

ALLOWED_KEYS = [
    POSITIONS_KEY, N_ATOMS_KEY, MASS_KEY, NEIGHBOR_LIST_KEY, TAG_KEY,
    DIRECTION_VECTORS_KEY, DISTANCES_KEY, EDGE_ATTRS_KEY, EDGE_EMBEDDING_KEY,
    CELL_KEY, PBC_KEY, NODE_FEATURES_KEY, NODE_ATTRS_KEY, ATOM_TYPE_KEY,
    ENERGY_KEY, FORCE_KEY, VELOCITY_KEY, BATCH_KEY,
]


def validate_keys(keys):
    for k in keys:
        if k not in ALLOWED_KEYS:
            raise KeyError(f"key {k!r} is not an AtomicData field ({ALLOWED_KEYS})")
