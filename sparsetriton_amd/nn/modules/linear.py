"""``SparseLinear`` (``sparsetriton/nn/modules/linear.py``): ``nn.Linear`` on the features."""

from torch import nn

from sparsetriton_amd.tensor import SparseTensor

__all__ = ["SparseLinear"]


class SparseLinear(nn.Linear):
    def forward(self, input):
        if isinstance(input, SparseTensor):
            return input.replace(super().forward(input.F))
        return super().forward(input)
