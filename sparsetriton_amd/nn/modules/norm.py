"""Normalisation layers (``sparsetriton/nn/modules/norm.py``).

``SparseBatchNorm`` has the reference's constructor, parameters and buffers
(``weight``, ``bias``, ``running_mean``, ``running_var``,
``num_batches_tracked``), so its state dict loads unchanged; its forward is
the per-sample batch normalisation of ``nn.functional.norm``.
``forward_act`` is the same layer with a residual add and ReLU fused into its
output pass, which the blocks use.  ``SparseLayerNorm`` is ``nn.LayerNorm`` on
the features, as in the reference.
"""

from typing import Optional

import torch
from torch import nn

from sparsetriton_amd.tensor import SparseTensor
from sparsetriton_amd.nn.functional.norm import sparse_batch_norm_act

__all__ = ["SparseBatchNorm", "SparseLayerNorm"]


class SparseBatchNorm(nn.Module):
    def __init__(self, num_features, eps=1e-5, momentum=0.1, affine=True, track_running_stats=True):
        super().__init__()
        self.num_features = num_features
        self.eps = eps
        self.momentum = momentum
        self.affine = affine
        self.track_running_stats = track_running_stats
        if affine:
            self.weight = nn.Parameter(torch.ones(num_features))
            self.bias = nn.Parameter(torch.zeros(num_features))
        else:
            self.register_parameter("weight", None)
            self.register_parameter("bias", None)
        if track_running_stats:
            self.register_buffer("running_mean", torch.zeros(num_features))
            self.register_buffer("running_var", torch.ones(num_features))
            self.register_buffer("num_batches_tracked", torch.tensor(0, dtype=torch.long))
        else:
            self.register_buffer("running_mean", None)
            self.register_buffer("running_var", None)
            self.register_buffer("num_batches_tracked", None)

    def reset_running_stats(self):
        if self.track_running_stats:
            self.running_mean.zero_()
            self.running_var.fill_(1)
            self.num_batches_tracked.zero_()

    def reset_parameters(self):
        self.reset_running_stats()
        if self.affine:
            self.weight.data.fill_(1.0)
            self.bias.data.zero_()

    def _check_input_dim(self, input):
        if input.F.dim() != 2:
            raise ValueError(f"Expected 2D input, got {input.F.dim()}D")

    def forward_act(self, input: SparseTensor, residual: Optional[SparseTensor] = None,
                    relu: bool = False) -> SparseTensor:
        """``act(self(input) + residual)`` in one pass (ReLU when ``relu``)."""
        self._check_input_dim(input)
        res = None
        if residual is not None:
            res = residual.F if isinstance(residual, SparseTensor) else residual
        out = sparse_batch_norm_act(input, self.weight, self.bias, self.running_mean, self.running_var,
                                    training=self.training, eps=self.eps, momentum=self.momentum, residual=res,
                                    relu=relu)
        if self.training and self.track_running_stats:
            self.num_batches_tracked += 1
        return out

    def forward(self, input: SparseTensor) -> SparseTensor:
        return self.forward_act(input)

    def folded(self):
        """(scale, shift), fp32 (C): evaluation-mode output = input * scale + shift."""
        scale = torch.rsqrt(self.running_var.detach().float() + self.eps)
        if self.weight is not None:
            scale = scale * self.weight.detach().float()
        shift = -self.running_mean.detach().float() * scale
        if self.bias is not None:
            shift = shift + self.bias.detach().float()
        return scale, shift


class SparseLayerNorm(nn.LayerNorm):
    def forward(self, input):
        if isinstance(input, SparseTensor):
            return input.replace(super().forward(input.F))
        return super().forward(input)
