from . import conv
from .conv import build_out_coords, compute_neighbor_indices, sparse_conv3d, sparse_conv3d_fused
from .norm import sparse_batch_norm, sparse_batch_norm_act
from .spatial import sparse_pooling, sparse_upsample

__all__ = ["conv", "sparse_conv3d", "sparse_conv3d_fused", "compute_neighbor_indices", "build_out_coords", "sparse_batch_norm",
           "sparse_batch_norm_act", "sparse_pooling", "sparse_upsample"]
