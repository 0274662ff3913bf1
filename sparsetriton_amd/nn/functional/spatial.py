"""Pooling and upsampling of sparse tensors (``sparsetriton/nn/functional/spatial.py:26-535``).

``sparse_pooling(input, kernel_size, padding, stride, mode)``: every input row
goes to the cell ``floor((coord + padding - kernel_size // 2) / stride)`` of
its sample; the output rows are the distinct cells in ascending
(b, x, y, z) order, each the max (``mode="max"``) or mean (``"avg"``) of its
rows; the new spatial shape is ``(s - kernel_size + 2 padding) // stride + 1``.
``sparse_upsample(input, scale_factor)``: each row becomes ``scale_factor**3``
rows at ``coord * scale_factor + (dx, dy, dz)``, dz fastest.  Both are HIP
kernels (``st_pool_*``, ``st_upsample*``) with autograd.

Deviation, documented: the reference packs the pooled cells through
``flatten_coord``'s 16-bit fields, which corrupts negative cells (an even
kernel with no padding sends coordinate 0 to cell -1); here cells are kept
exact, so negative cells stay negative.  Cells outside int16 (or samples
outside [0, 32767]) raise ``ValueError``.
"""

import ctypes
from typing import Tuple

import torch

from sparsetriton_amd import _lib
from sparsetriton_amd.tensor import SparseTensor

__all__ = ["sparse_pooling", "sparse_upsample"]

_MODES = {"max": 0, "avg": 1}


class _Pool(torch.autograd.Function):
    @staticmethod
    def forward(ctx, feats, coords, kernel_size, padding, stride, mode):
        x = feats.contiguous()
        c = coords.contiguous()
        n, C = x.shape
        dev = x.device
        s = _lib.stream_of(dev)
        nbytes = ctypes.c_size_t()
        _lib.call("st_pool_workspace", n, ctypes.byref(nbytes))
        ws = torch.empty((max(nbytes.value, 1),), dtype=torch.uint8, device=dev)
        perm = torch.empty((max(n, 1),), dtype=torch.int32, device=dev)
        seg = torch.empty((n + 1,), dtype=torch.int32, device=dev)
        inv = torch.empty((max(n, 1),), dtype=torch.int32, device=dev)
        oc = torch.empty((max(n, 1), 4), dtype=c.dtype, device=dev)
        counts = torch.empty((2,), dtype=torch.int32, device=dev)
        _lib.call("st_pool_plan", _lib.ptr(c), _lib.coord_code(c.dtype), n, int(kernel_size), int(stride),
                  int(padding), _lib.ptr(ws), nbytes.value, _lib.ptr(perm), _lib.ptr(seg), _lib.ptr(inv),
                  _lib.ptr(oc), _lib.ptr(counts), s)
        n_out, bad = counts.tolist()
        if bad:
            raise ValueError(f"{bad} pooled cells fall outside the coordinate key range "
                             "(sample index in [0, 32767], spatial values in int16)")
        out = torch.empty((n_out, C), dtype=x.dtype, device=dev)
        _lib.call("st_pool_forward", _lib.ptr(x), C, _lib.feat_code(x.dtype), _lib.ptr(perm), _lib.ptr(seg), n_out,
                  _MODES[mode], _lib.ptr(out), s)
        ctx.save_for_backward(x if mode == "max" else None, out if mode == "max" else None, inv, seg)
        ctx.meta = (n, C, _MODES[mode])
        ctx.mark_non_differentiable(oc)
        return out, oc[:n_out]

    @staticmethod
    def backward(ctx, dout, _dcoords):
        x, out, inv, seg = ctx.saved_tensors
        n, C, mode = ctx.meta
        g = dout.contiguous()
        dfeats = torch.empty((n, C), dtype=g.dtype, device=g.device)
        _lib.call("st_pool_backward", _lib.ptr(x), _lib.ptr(out), _lib.ptr(g), n, C, _lib.feat_code(g.dtype),
                  _lib.ptr(inv), _lib.ptr(seg), mode, _lib.ptr(dfeats), _lib.stream_of(g.device))
        return dfeats, None, None, None, None, None


def sparse_pooling(input: SparseTensor, kernel_size: int, padding: int, stride: int, mode: str) -> SparseTensor:
    if mode not in _MODES:
        raise ValueError(f"Unsupported mode: {mode}")
    _lib.require_device(input.F, "SparseTensor features")
    if stride is None:
        stride = kernel_size
    new_shape = tuple((int(s) - kernel_size + padding * 2) // stride + 1 for s in input.spatial_shape)
    feats, coords = _Pool.apply(input.F, input.C, kernel_size, padding, stride, mode)
    return SparseTensor(feats, coords, spatial_shape=new_shape, batch_size=input.batch_size)


class _Upsample(torch.autograd.Function):
    @staticmethod
    def forward(ctx, feats, coords, scale):
        x = feats.contiguous()
        c = coords.contiguous()
        n, C = x.shape
        s3 = scale ** 3
        out = torch.empty((n * s3, C), dtype=x.dtype, device=x.device)
        oc = torch.empty((n * s3, 4), dtype=c.dtype, device=x.device)
        _lib.call("st_upsample", _lib.ptr(x), _lib.ptr(c), _lib.coord_code(c.dtype), n, C, _lib.feat_code(x.dtype),
                  int(scale), _lib.ptr(out), _lib.ptr(oc), _lib.stream_of(x.device))
        ctx.meta = (n, C, int(scale))
        ctx.mark_non_differentiable(oc)
        return out, oc

    @staticmethod
    def backward(ctx, dout, _dcoords):
        n, C, scale = ctx.meta
        g = dout.contiguous()
        dfeats = torch.empty((n, C), dtype=g.dtype, device=g.device)
        _lib.call("st_upsample_backward", _lib.ptr(g), n, C, _lib.feat_code(g.dtype), scale, _lib.ptr(dfeats),
                  _lib.stream_of(g.device))
        return dfeats, None, None


def sparse_upsample(input: SparseTensor, scale_factor: int = None) -> SparseTensor:
    if scale_factor is None or int(scale_factor) < 1:
        raise ValueError(f"scale_factor must be a positive integer, got {scale_factor}")
    _lib.require_device(input.F, "SparseTensor features")
    feats, coords = _Upsample.apply(input.F, input.C, int(scale_factor))
    new_shape = tuple(int(s) * int(scale_factor) for s in input.spatial_shape)
    return SparseTensor(feats, coords, spatial_shape=new_shape, batch_size=input.batch_size)
