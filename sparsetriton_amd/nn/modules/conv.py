"""Sparse convolution modules (``sparsetriton/nn/modules/conv.py:31-365``).

``SubMConv3D``, ``SparseConv3D`` and ``SparseConvTransposed3D`` keep the
reference's constructor arguments, attribute names and parameter layout:
``weight`` (k^3, C_in, C_out) and ``bias`` (C_out), both initialised
U(-1/sqrt(C_in * k^3), +1/sqrt(C_in * k^3)), so reference checkpoints load
unchanged through ``state_dict``.
"""

import math
from typing import Tuple, Union

import torch
from torch import nn

from sparsetriton_amd.tensor import SparseTensor
from sparsetriton_amd.nn.functional.conv.conv import sparse_conv3d, sparse_conv3d_fused
from sparsetriton_amd.utils.utils import make_ntuple

__all__ = ["SparseConv3DBase", "SparseConv3D", "SubMConv3D", "SparseConvTransposed3D"]


class SparseConv3DBase(nn.Module):
    """Common parameters and forward of the sparse convolution layers."""

    def __init__(
        self,
        in_channels: int,
        out_channels: int,
        kernel_size: Union[int, Tuple[int, int, int]] = 3,
        stride: Union[int, Tuple[int, int, int]] = 1,
        padding: Union[int, Tuple[int, int, int]] = 0,
        dilation: Union[int, Tuple[int, int, int]] = 1,
        subm: bool = True,
        bias: bool = True,
        transposed: bool = False,
    ):
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = make_ntuple(kernel_size, 3)
        self.stride = make_ntuple(stride, 3)
        self.padding = make_ntuple(padding, 3)
        self.dilation = make_ntuple(dilation, 3)
        self.subm = subm
        self.transposed = transposed
        self.kernel_volume = self.kernel_size[0] * self.kernel_size[1] * self.kernel_size[2]
        self.weight = nn.Parameter(torch.empty(self.kernel_volume, in_channels, out_channels))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_channels))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        bound = 1.0 / math.sqrt(self.in_channels * self.kernel_volume)
        self.weight.data.uniform_(-bound, bound)
        if self.bias is not None:
            self.bias.data.uniform_(-bound, bound)

    def forward(self, input: SparseTensor) -> SparseTensor:
        return sparse_conv3d(
            tensor=input,
            weight=self.weight,
            kernel_size=self.kernel_size,
            bias=self.bias,
            stride=self.stride,
            dilation=self.dilation,
            padding=self.padding,
            submanifold=self.subm,
            transposed=self.transposed,
        )


    def forward_fused(self, input: SparseTensor, scale=None, shift=None, residual=None,
                      relu: bool = False) -> SparseTensor:
        """Inference forward with ``act((conv + bias) * scale + shift + residual)`` fused into the
        GEMM's store (see ``sparse_conv3d_fused``)."""
        return sparse_conv3d_fused(
            input, self.weight, self.kernel_size, bias=self.bias, stride=self.stride, dilation=self.dilation,
            padding=self.padding, transposed=self.transposed, submanifold=self.subm, scale=scale, shift=shift,
            residual=residual, relu=relu)


class SparseConv3D(SparseConv3DBase):
    """Strided (generalised) sparse convolution; output coordinates are all reachable sites."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size=3, stride=1, padding=0, dilation=1,
                 bias: bool = True):
        super().__init__(in_channels, out_channels, kernel_size=kernel_size, stride=stride, padding=padding,
                         dilation=dilation, bias=bias, subm=False, transposed=False)


class SubMConv3D(SparseConv3DBase):
    """Submanifold sparse convolution: output sites = input sites."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size=3, stride=1, dilation=1, bias: bool = True):
        super().__init__(in_channels, out_channels, kernel_size=kernel_size, stride=stride, dilation=dilation,
                         bias=bias, subm=True, transposed=False)


class SparseConvTransposed3D(SparseConv3DBase):
    """Transposed sparse convolution (upsampling); ``subm`` / ``transposed`` args kept for compatibility."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size=3, stride=1, padding=0, dilation=1,
                 subm: bool = True, bias: bool = True, transposed: bool = False):
        super().__init__(in_channels, out_channels, kernel_size=kernel_size, stride=stride, padding=padding,
                         dilation=dilation, bias=bias, subm=False, transposed=True)
