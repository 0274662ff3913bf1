"""``mask_spatial_range`` (``sparsetriton/utils/spatial/tile.py:16-85``): which coordinate rows lie
inside inclusive (min, max) limits on x, y and z (``None`` = unbounded), as a bool tensor; one HIP
kernel (``st_mask_spatial_range``)."""

import ctypes

import torch

from sparsetriton_amd import _lib

__all__ = ["mask_spatial_range"]


def mask_spatial_range(coords: torch.Tensor, x_lim: tuple = (None, None), y_lim: tuple = (None, None),
                       z_lim: tuple = (None, None)) -> torch.Tensor:
    n = coords.shape[0]
    mask = torch.empty((n,), dtype=torch.bool, device=coords.device)
    if n == 0:
        return mask
    _lib.require_device(coords, "coordinates")
    info = torch.iinfo(coords.dtype)
    lims = []
    for lo, hi in (x_lim, y_lim, z_lim):
        lims += [int(lo) if lo is not None else info.min, int(hi) if hi is not None else info.max]
    c = coords.contiguous()
    arr = (ctypes.c_int64 * 6)(*lims)
    _lib.call("st_mask_spatial_range", _lib.ptr(c), _lib.coord_code(c.dtype), n, arr, _lib.ptr(mask),
              _lib.stream_of(c.device))
    return mask
