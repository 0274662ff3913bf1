"""Sparse -> dense conversion (``sparsetriton/utils/to_dense.py:30-282``).

``to_dense(feats, coords, spatial_range)`` returns the channels-last grid
(B, X, Y, Z, C), B = max batch index + 1, holding row r of ``feats`` at the
cell of ``coords[r]`` and zeros elsewhere; it is differentiable in ``feats``
(the gradient gathers the grid's gradient at the same cells).  Both directions
are HIP kernels (``st_to_dense`` / ``st_from_dense``); coordinates outside
the grid are skipped.  As in the reference, the tensors must be on the GPU.
"""

from typing import Tuple

import torch

from sparsetriton_amd import _lib

__all__ = ["to_dense"]


class _ToDense(torch.autograd.Function):
    @staticmethod
    def forward(ctx, feats, coords, spatial_range, batch_size):
        x = feats.contiguous()
        c = coords.contiguous()
        n, C = x.shape
        B = int(batch_size)
        sx, sy, sz = (int(v) for v in spatial_range)
        out = torch.empty((B, sx, sy, sz, C), dtype=x.dtype, device=x.device)
        _lib.call("st_to_dense", _lib.ptr(x), n, C, _lib.feat_code(x.dtype), _lib.ptr(c), _lib.coord_code(c.dtype),
                  B, sx, sy, sz, _lib.ptr(out), _lib.stream_of(x.device))
        ctx.save_for_backward(c)
        ctx.geom = (B, sx, sy, sz, n, C)
        return out

    @staticmethod
    def backward(ctx, grad):
        (c,) = ctx.saved_tensors
        B, sx, sy, sz, n, C = ctx.geom
        g = grad.contiguous()
        dfeats = torch.empty((n, C), dtype=g.dtype, device=g.device)
        _lib.call("st_from_dense", _lib.ptr(g), B, sx, sy, sz, C, _lib.feat_code(g.dtype), _lib.ptr(c),
                  _lib.coord_code(c.dtype), n, _lib.ptr(dfeats), _lib.stream_of(g.device))
        return dfeats, None, None, None


def to_dense(feats: torch.Tensor, coords: torch.Tensor, spatial_range: Tuple[int]) -> torch.Tensor:
    _lib.require_device(feats, "features")
    if isinstance(spatial_range, torch.Size):
        spatial_range = tuple(spatial_range)
    spatial_range = tuple(int(s) for s in spatial_range)
    assert len(spatial_range) == 3, "spatial_range must be (X, Y, Z)"
    assert coords.ndim == 2 and coords.shape[1] == 4 and coords.shape[0] == feats.shape[0], \
        "coords must be (N, 4) with N = feats rows"
    batch_size = 1 if coords.shape[0] == 0 else int(coords[:, 0].max().item()) + 1
    coords = coords.to(device=feats.device)
    if coords.dtype not in _lib.COORD_DTYPES:
        coords = coords.to(torch.int32)
    return _ToDense.apply(feats, coords, spatial_range, batch_size)
