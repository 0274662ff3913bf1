"""Sparse -> dense scatter, used to compare against dense convolution.

Same contract as the reference (``sparsetriton/utils/to_dense.py:242-282``):
``to_dense(feats, coords, spatial_range)`` returns a channels-last tensor of
shape (B, X, Y, Z, C) with B = max batch index + 1, differentiable in
``feats``.  This is the test bridge to dense ``conv3d``, not part of the
convolution path, so it is a plain torch indexed write.
"""

from typing import Tuple

import torch

__all__ = ["to_dense"]


def to_dense(feats: torch.Tensor, coords: torch.Tensor, spatial_range: Tuple[int]) -> torch.Tensor:
    if isinstance(spatial_range, torch.Size):
        spatial_range = tuple(spatial_range)
    spatial_range = tuple(int(s) for s in spatial_range)
    batch_size = 1 if coords.shape[0] == 0 else int(coords[:, 0].max().item()) + 1
    out = torch.zeros((batch_size,) + spatial_range + (feats.shape[1],), dtype=feats.dtype, device=feats.device)
    if coords.shape[0] == 0:
        return out
    c = coords.long()
    return out.index_put((c[:, 0], c[:, 1], c[:, 2], c[:, 3]), feats)
