"""Convolution blocks (``sparsetriton/nn/modules/blocks.py:21-124``).

Each block has the reference's children in the reference's order, so state
dicts load unchanged:

* ``SparseConvBlock``: ``SubMConv3D`` (with the block's stride), ``SparseBatchNorm``, ``ReLU``;
* ``SparseConvTransposeBlock``: ``SparseConvTransposed3D``, ``SparseBatchNorm``, ``ReLU``;
* ``SparseResBlock``: ``main`` = SubM conv, BN, ReLU, SubM conv, BN; ``shortcut`` = identity,
  or a 1x1x1 SubM conv with the stride and a BN when the channels or the stride change;
  output ``relu(main(x) + shortcut(x))``.

The forward passes fuse each batch norm with the ReLU after it, and the
residual block's last batch norm with the residual add and the final ReLU,
into one output pass (``SparseBatchNorm.forward_act``).  In evaluation under
``torch.no_grad()`` with the precomputed-map algorithm, the batch norm (its
running statistics folded to one affine map per channel), the residual add and
the ReLU go into the convolution GEMM's store instead (``forward_fused``), so a
block is one kernel pass per convolution.  A block whose children were replaced
by other modules runs them one after another.
"""

from typing import List, Tuple, Union

import numpy as np
from torch import nn

import torch

from sparsetriton_amd.config import ConvAlgo, get_conv_algo
from sparsetriton_amd.tensor import SparseTensor
from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import tiled_ok
from sparsetriton_amd.nn.modules.conv import SparseConv3DBase, SparseConvTransposed3D, SubMConv3D
from sparsetriton_amd.nn.modules.norm import SparseBatchNorm
from sparsetriton_amd.nn.modules.activation import ReLU

__all__ = ["SparseConvBlock", "SparseConvTransposeBlock", "SparseResBlock"]


def _fusable(bn, act) -> bool:
    return type(bn) is SparseBatchNorm and type(act) is ReLU


def _store_fusable(conv, bn, x: SparseTensor) -> bool:
    """Whether conv + evaluation-mode bn can run as one GEMM with a store epilogue."""
    return (isinstance(conv, SparseConv3DBase) and type(bn) is SparseBatchNorm and not bn.training
            and bn.track_running_stats and not torch.is_grad_enabled()
            and get_conv_algo() == ConvAlgo.PrecomputedNeighborGEMM and x.F.is_cuda
            and tiled_ok(x.F.dtype, x.F.shape[1]))


class _ConvBnReLU(nn.Sequential):
    def forward(self, x: SparseTensor) -> SparseTensor:
        if len(self) == 3 and _fusable(self[1], self[2]):
            if _store_fusable(self[0], self[1], x):
                scale, shift = self[1].folded()
                return self[0].forward_fused(x, scale, shift, relu=True)
            return self[1].forward_act(self[0](x), relu=True)
        return super().forward(x)


class SparseConvBlock(_ConvBnReLU):
    def __init__(
        self,
        in_channels: int,
        out_channels: int,
        kernel_size: Union[int, List[int], Tuple[int, ...]],
        stride: Union[int, List[int], Tuple[int, ...]] = 1,
        dilation: int = 1,
    ) -> None:
        super().__init__(
            SubMConv3D(in_channels, out_channels, kernel_size, stride=stride, dilation=dilation),
            SparseBatchNorm(out_channels),
            ReLU(inplace=True),
        )


class SparseConvTransposeBlock(_ConvBnReLU):
    def __init__(
        self,
        in_channels: int,
        out_channels: int,
        kernel_size: Union[int, List[int], Tuple[int, ...]],
        stride: Union[int, List[int], Tuple[int, ...]] = 1,
        dilation: int = 1,
    ) -> None:
        super().__init__(
            SparseConvTransposed3D(in_channels, out_channels, kernel_size, stride=stride, dilation=dilation),
            SparseBatchNorm(out_channels),
            ReLU(inplace=True),
        )


class SparseResBlock(nn.Module):
    def __init__(
        self,
        in_channels: int,
        out_channels: int,
        kernel_size: Union[int, List[int], Tuple[int, ...]],
        stride: Union[int, List[int], Tuple[int, ...]] = 1,
        dilation: int = 1,
    ) -> None:
        super().__init__()
        self.main = nn.Sequential(
            SubMConv3D(in_channels, out_channels, kernel_size, dilation=dilation, stride=stride),
            SparseBatchNorm(out_channels),
            ReLU(inplace=True),
            SubMConv3D(out_channels, out_channels, kernel_size, dilation=dilation),
            SparseBatchNorm(out_channels),
        )
        if in_channels != out_channels or np.prod(stride) != 1:
            self.shortcut = nn.Sequential(
                SubMConv3D(in_channels, out_channels, 1, stride=stride),
                SparseBatchNorm(out_channels),
            )
        else:
            self.shortcut = nn.Identity()
        self.relu = ReLU(inplace=True)

    def forward(self, x: SparseTensor) -> SparseTensor:
        m = self.main
        if len(m) == 5 and _fusable(m[1], m[2]) and type(m[4]) is SparseBatchNorm and type(self.relu) is ReLU:
            if self._store_fused_ok(x):
                h = m[0].forward_fused(x, *m[1].folded(), relu=True)
                if isinstance(self.shortcut, nn.Identity):
                    sc = x.F
                else:
                    sc = self.shortcut[0].forward_fused(x, *self.shortcut[1].folded()).F
                if sc.shape != (h.F.shape[0], m[3].out_channels):
                    raise RuntimeError(f"residual shapes differ: main {(h.F.shape[0], m[3].out_channels)}, "
                                       f"shortcut {tuple(sc.shape)}")
                return m[3].forward_fused(h, *m[4].folded(), residual=sc.to(h.F.dtype), relu=True)
            h = m[1].forward_act(m[0](x), relu=True)
            h = m[3](h)
            sc = self.shortcut(x)
            if sc.F.shape != h.F.shape:
                raise RuntimeError(f"residual shapes differ: main {tuple(h.F.shape)}, shortcut {tuple(sc.F.shape)}")
            return m[4].forward_act(h, residual=sc.F.to(h.F.dtype), relu=True)
        return self.relu(self.main(x) + self.shortcut(x))

    def _store_fused_ok(self, x: SparseTensor) -> bool:
        m = self.main
        if not (_store_fusable(m[0], m[1], x) and _store_fusable(m[3], m[4], x)):
            return False
        if m[3].in_channels != m[0].out_channels or not tiled_ok(x.F.dtype, m[3].in_channels):
            return False
        sc = self.shortcut
        return isinstance(sc, nn.Identity) or (len(sc) == 2 and _store_fusable(sc[0], sc[1], x))
