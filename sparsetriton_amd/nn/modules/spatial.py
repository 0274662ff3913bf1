"""Pooling / upsampling / downsampling layers (``sparsetriton/nn/modules/spatial.py``)."""

from typing import Literal

from torch import nn

from sparsetriton_amd.tensor import SparseTensor
from sparsetriton_amd.nn.functional.spatial import sparse_pooling, sparse_upsample

__all__ = ["SparsePooling", "SparseUpsample", "SparseDownsample"]


class SparsePooling(nn.Module):
    def __init__(self, kernel_size: int, mode: Literal["avg", "max"] = "avg", stride: int = 1, padding: int = 0):
        super().__init__()
        if mode not in ["avg", "max"]:
            raise ValueError(f"mode must be 'avg' or 'max', got '{mode}'")
        self.kernel_size = kernel_size
        self.stride = stride
        self.mode = mode
        self.padding = padding

    def forward(self, x: SparseTensor) -> SparseTensor:
        return sparse_pooling(x, self.kernel_size, self.padding, self.stride, self.mode)


class SparseUpsample(nn.Module):
    def __init__(self, scale_factor: int = None):
        super().__init__()
        self.scale_factor = scale_factor

    def forward(self, input: SparseTensor) -> SparseTensor:
        return sparse_upsample(input, self.scale_factor)


class SparseDownsample(SparsePooling):
    """Pooling with kernel_size = stride = scale_factor and no padding."""

    def __init__(self, scale_factor: int = None, mode: Literal["max", "avg"] = "max"):
        super().__init__(kernel_size=scale_factor, stride=scale_factor, mode=mode, padding=0)
