"""Coordinate hash table, dense conversion and argument helpers."""

from .hash import HashTable, flatten_coord, hash_coords, unflatten_coord
from .to_dense import to_dense
from .utils import make_ntuple
from .spatial import mask_spatial_range

__all__ = ["HashTable", "flatten_coord", "hash_coords", "unflatten_coord", "to_dense", "make_ntuple",
           "mask_spatial_range"]
