"""Elementwise activations on sparse features (``sparsetriton/nn/modules/activation.py``).

As in the reference, each is the ``torch.nn`` module applied to ``tensor.F``
with the coordinates kept.  (The blocks fuse their ReLU into the preceding
batch normalisation's output pass instead.)
"""

from torch import nn

from sparsetriton_amd.tensor import SparseTensor

__all__ = ["ReLU", "LeakyReLU", "SiLU", "GELU", "Sigmoid", "Tanh"]


def _sparse_forward(base):
    def forward(self, input):
        if isinstance(input, SparseTensor):
            return input.replace(base.forward(self, input.F))
        return base.forward(self, input)

    return forward


class ReLU(nn.ReLU):
    forward = _sparse_forward(nn.ReLU)


class LeakyReLU(nn.LeakyReLU):
    forward = _sparse_forward(nn.LeakyReLU)


class SiLU(nn.SiLU):
    forward = _sparse_forward(nn.SiLU)


class GELU(nn.GELU):
    forward = _sparse_forward(nn.GELU)


class Sigmoid(nn.Sigmoid):
    forward = _sparse_forward(nn.Sigmoid)


class Tanh(nn.Tanh):
    forward = _sparse_forward(nn.Tanh)
