from .conv import compute_neighbor_indices, sparse_conv3d, sparse_conv3d_fused
from .kmap import KernelMap, build_out_coords

__all__ = ["sparse_conv3d", "sparse_conv3d_fused", "compute_neighbor_indices", "build_out_coords", "KernelMap"]
