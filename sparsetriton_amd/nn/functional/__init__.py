from . import conv
from .conv import build_out_coords, compute_neighbor_indices, sparse_conv3d

__all__ = ["conv", "sparse_conv3d", "compute_neighbor_indices", "build_out_coords"]
