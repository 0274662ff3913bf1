from .conv import SparseConv3D, SparseConv3DBase, SparseConvTransposed3D, SubMConv3D
from .activation import GELU, LeakyReLU, ReLU, SiLU, Sigmoid, Tanh
from .linear import SparseLinear
from .norm import SparseBatchNorm, SparseLayerNorm
from .blocks import SparseConvBlock, SparseConvTransposeBlock, SparseResBlock
from .spatial import SparseDownsample, SparsePooling, SparseUpsample

__all__ = [
    "SparseConv3DBase", "SparseConv3D", "SubMConv3D", "SparseConvTransposed3D",
    "ReLU", "LeakyReLU", "SiLU", "GELU", "Sigmoid", "Tanh",
    "SparseLinear", "SparseBatchNorm", "SparseLayerNorm",
    "SparseConvBlock", "SparseConvTransposeBlock", "SparseResBlock",
    "SparsePooling", "SparseUpsample", "SparseDownsample",
]
