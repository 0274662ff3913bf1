"""Implicit GEMM that probes the coordinate hash table inside the kernel.

``ConvHashOnTheFlyImplicitGEMM.apply(features, weights, coords, kernel_offsets,
table_keys, table_vals, spatial_shape, lookup_stride)`` keeps the reference's
signature and meaning (``.../conv/funcs/implicit_hashfly_gemm.py:330-452``):
output row o with coordinate c sums, over offsets k, features at
``q = c * lookup_stride - kernel_offsets[k]`` (when 0 <= q < spatial_shape
and q is in the table) times ``weights[k]``.  ``table_keys`` /
``table_vals`` are a ``HashTable``'s arrays (exact int64 keys here).

No kernel map is stored.  The probe runs once per destination-row tile and
offset (the reference repeats it for every C_out tile).  Two optional
trailing arguments make the backward a gather like the forward:
``in_coords`` (rows of ``features``) and ``grad_lookup`` (an
``InputGradLookup``: a table of the output coordinates and the rule that
finds them from an input row).  Given both, the input gradient probes that
table; without them it builds the transposed map once from the forward
lookups.  The weight gradient probes the input table once per (row, offset)
into a map that lives only for the backward call and walks its pair list.

``ConvSubmFlyGEMM`` is the same algorithm for a submanifold convolution with
the lookups in the coordinates' brick index (``BrickIndex``) instead of the
table: the index answers a lookup from L2 in three dependent loads where a
table probe reads a random line of a table several times larger, and the
GEMM's prologue looks up its whole tile before the MFMA loop, skipping
offsets none of the tile's rows has.
"""

import ctypes
import os
from typing import Optional

import torch

from sparsetriton_amd import _lib
from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import (
    _concurrent_backward,
    _side_stream,
    gather_gemm,
    weight_prep,
    wgrad,
    wgrad_buffers,
    wgrad_splits,
)
from sparsetriton_amd.nn.functional.conv.kmap import BrickIndex, KernelMap, row_representatives

__all__ = ["ConvHashOnTheFlyImplicitGEMM", "ConvSubmFlyGEMM", "InputGradLookup", "fly_tile_order", "subm_fly_ok"]


def _lookup(K: int, sign: int, mul: int, div: int, bounds, row_bounds=(0, 0, 0)) -> _lib.Lookup:
    lk = _lib.Lookup()
    lk.K, lk.sign, lk.mul, lk.div = K, sign, int(mul), int(div)
    for a in range(3):
        lk.bounds[a] = int(bounds[a])
        lk.row_bounds[a] = int(row_bounds[a])
    return lk


def _as_u64_keys(table_keys: torch.Tensor) -> torch.Tensor:
    assert table_keys.dtype == torch.int64, "table_keys must be this package's int64 packed-coordinate keys"
    return table_keys


def hashfly_gemm(A, dst_coords, offsets_i32, lk, keys, vals, Bt, n_dst):
    Kd, Nd = A.shape[1], Bt.shape[1]
    out = torch.empty((n_dst, Nd), dtype=A.dtype, device=A.device)
    _lib.call("st_hashfly_gemm", _lib.ptr(A), A.shape[0], _lib.ptr(dst_coords), _lib.coord_code(dst_coords.dtype),
              n_dst, _lib.ptr(offsets_i32), ctypes.byref(lk), _lib.ptr(keys), _lib.ptr(vals), keys.shape[0],
              _lib.ptr(Bt), None, _lib.ptr(out), Kd, Nd, _lib.compute_code(A.dtype), _lib.stream_of(A.device))
    return out


def hashfly_wgrad_probing(X, dY, out_coords, offsets_i32, lk, keys, vals, dw_dtype):
    """Weight gradient probing the table inside the kernel (``st_hashfly_wgrad``): one probe per
    (row, offset) per row split, partials per (offset, split)."""
    K, C_in, C_out = lk.K, X.shape[1], dY.shape[1]
    n_out = out_coords.shape[0]
    splits = wgrad_splits(n_out)
    partials = torch.empty((K * splits * C_in * C_out,), dtype=torch.float32, device=X.device)
    dW = torch.empty((K, C_in, C_out), dtype=dw_dtype, device=X.device)
    _lib.call("st_hashfly_wgrad", _lib.ptr(X), X.shape[0], _lib.ptr(dY), _lib.ptr(out_coords),
              _lib.coord_code(out_coords.dtype),
              n_out, _lib.ptr(offsets_i32), ctypes.byref(lk), _lib.ptr(keys), _lib.ptr(vals), keys.shape[0], C_in,
              C_out, _lib.feat_code(X.dtype), _lib.ptr(partials), splits, _lib.ptr(dW), _lib.feat_code(dw_dtype),
              _lib.stream_of(X.device))
    return dW


class InputGradLookup:
    """How the input gradient finds the output rows an input row feeds.

    Forward pairs satisfy ``out * s - t_k = in_key``; solved for the output:
    ``out = (in * mul + t_k) / div``, looked up in ``table_keys`` /
    ``table_values`` (a table of the output coordinates).  Input rows outside
    ``in_shape`` have no forward pairs; the output is not bounded (a
    submanifold output row outside ``out_shape`` still takes its in-bounds
    neighbours in the forward).

      submanifold / stride 1 : mul 1, div 1, table = input table
      strided (s)            : mul 1, div s, table = output dedup table
      transposed (s)         : mul s, div 1, table = output dedup table

    The rule finds one output row per coordinate and assumes each input
    coordinate is one row: with repeated input coordinates the forward reads
    only the lowest of them, so the lookup is disabled (``usable()`` False)
    when ``duplicate_check`` -- a StatusSnapshot of the input table -- counts
    any, and the input gradient takes the transposed-map path instead.
    """

    def __init__(self, table_keys, table_values, mul: int, div: int, out_shape, in_shape, duplicate_check=None):
        self.table_keys, self.table_values = table_keys, table_values
        self.mul, self.div = int(mul), int(div)
        self.out_shape = tuple(int(v) for v in out_shape)
        self.in_shape = tuple(int(v) for v in in_shape)
        self._check = duplicate_check
        self._usable = True

    def usable(self) -> bool:
        if self._check is not None:
            self._usable = self._check.counters()["duplicate"] == 0
            self._check = None
        return self._usable


class ConvHashOnTheFlyImplicitGEMM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, features, weights, coords, kernel_offsets, hash_table_keys, hash_table_vals, spatial_shape,
                lookup_stride, in_coords=None, grad_lookup=None):
        _lib.require_device(features, "features")
        N_in, C_in = features.shape
        K, C_in_w, C_out = weights.shape
        assert C_in_w == C_in, f"weights C_in ({C_in_w}) != features C_in ({C_in})"
        assert kernel_offsets.shape[0] == K, "kernel_offsets rows must equal the kernel volume"
        features = features.contiguous()
        coords = coords.contiguous()
        offs = kernel_offsets.to(torch.int32).contiguous()
        keys = _as_u64_keys(hash_table_keys)
        vals = hash_table_vals.contiguous()
        shape = tuple(int(v) for v in spatial_shape)
        lk = _lookup(K, -1, int(lookup_stride), 1, shape)
        wt = weight_prep(weights.to(features.dtype).contiguous(), _lib.W_TRANSPOSE)
        out = hashfly_gemm(features, coords, offs, lk, keys, vals, wt, coords.shape[0])
        ctx.save_for_backward(features, weights, coords, offs, keys, vals)
        ctx.shape = shape
        ctx.lookup_stride = int(lookup_stride)
        ctx.in_coords = in_coords
        ctx.grad_lookup = grad_lookup
        return out

    @staticmethod
    def backward(ctx, grad_output):
        features, weights, coords, offs, keys, vals = ctx.saved_tensors
        K = weights.shape[0]
        N_in = features.shape[0]
        grad_output = grad_output.to(features.dtype).contiguous()
        s = ctx.lookup_stride
        grad_input = grad_weights = None
        n_out = coords.shape[0]
        probes = []  # the forward's lookups, probed once into a map that lives until this function returns

        def probed_map() -> torch.Tensor:
            if not probes:
                nbr = torch.empty((K, n_out), dtype=torch.int32, device=coords.device)
                _lib.call("st_kmap_query", _lib.ptr(coords), _lib.coord_code(coords.dtype), n_out,
                          _lib.ptr(offs), K, s, *ctx.shape, _lib.ptr(keys), _lib.ptr(vals), keys.shape[0],
                          _lib.ptr(nbr), n_out, 1, None, None, _lib.stream_of(coords.device))
                probes.append(nbr)
            return probes[0]

        if ctx.needs_input_grad[0]:
            w = weights.to(features.dtype).contiguous()
            gl = ctx.grad_lookup
            if ctx.in_coords is not None and gl is not None and gl.usable():
                lk = _lookup(K, +1, gl.mul, gl.div, (0, 0, 0), gl.in_shape)
                grad_input = hashfly_gemm(grad_output, ctx.in_coords.contiguous(), offs, lk, gl.table_keys,
                                          gl.table_values, w, N_in)
            else:
                kmap = KernelMap(probed_map(), N_in, n_out, K)
                kmap.set_row_representatives(row_representatives(coords))  # repeated output coordinates
                kmap.ensure_inverse()
                grad_input = gather_gemm(kmap.fold_output_rows(grad_output), kmap.invnbr, N_in, 1, kmap.in_masks,
                                         w, N_in, K)
        if ctx.needs_input_grad[1]:
            # One probe per (row, offset) into the map above, compacted into the (offset, output)-sorted
            # pair list the pair-list weight gradient walks: a probe inside the weight-gradient kernel
            # would be repeated for every C_in x C_out tile and leaves its MFMAs waiting on the probes.
            kmap = KernelMap(probed_map(), N_in, n_out, K)
            grad_weights = wgrad(features, grad_output, kmap, weights.dtype,
                                 pairs=kmap.pair_list(with_tiles=False))
        return grad_input, grad_weights, None, None, None, None, None, None, None, None


def subm_fly_ok(n: int, C_in: int, C_out: int, K: int, dtype: torch.dtype) -> bool:
    """Whether ``st_subm_fly_gemm`` takes both directions of a C_in -> C_out convolution over ``n``
    rows: the shape is built and the operands of the forward (n x C_in) and of the input gradient
    (n x C_out) fit the kernel's 32-bit buffer offsets.  Otherwise the convolution runs on the
    table-probing kernels."""
    code = _lib.compute_code(dtype)
    lib = _lib.lib()
    return bool(lib.st_subm_fly_ok(n, C_in, C_out, K, code)) and bool(lib.st_subm_fly_ok(n, C_out, C_in, K, code))


def subm_fly_gemm(A: torch.Tensor, index: BrickIndex, offsets_i32: torch.Tensor, Bt: torch.Tensor,
                  order: Optional[torch.Tensor] = None, reverse_k: bool = False) -> torch.Tensor:
    """out[r] = sum_k A[nbr(k, r)] @ Bt[k]^T over the submanifold neighbours found in ``index``
    (``Bt[K-1-k]`` with ``reverse_k``), 128-row tiles taken in ``order`` (``index.tile_order``)
    when given, else in row order; the sums are the same either way."""
    n, Kd, Nd = index.n, A.shape[1], Bt.shape[1]
    out = torch.empty((n, Nd), dtype=A.dtype, device=A.device)
    _lib.call("st_subm_fly_gemm", _lib.ptr(A), _lib.ptr(index.coords), _lib.coord_code(index.coords.dtype), n,
              _lib.ptr(offsets_i32), offsets_i32.shape[0], *index.geometry, _lib.ptr(index.work), index.nbytes,
              _lib.ptr(order) if order is not None else None, _lib.ptr(Bt), None, _lib.ptr(out), Kd, Nd,
              _lib.compute_code(A.dtype), _lib.GATHER_REVERSE_K if reverse_k else 0, _lib.stream_of(A.device))
    return out


def fly_tile_order(index: BrickIndex, kernel_offsets: torch.Tensor, key) -> Optional[torch.Tensor]:
    """The index's mask-sorted tile order for the fly GEMMs (``BrickIndex.tile_order``);
    ``ST_FLY_ORDER=0`` keeps the rows' own order (for timing the two against each other)."""
    if os.environ.get("ST_FLY_ORDER", "1") == "0":
        return None
    return index.tile_order(kernel_offsets, key)


class ConvSubmFlyGEMM(torch.autograd.Function):
    """Submanifold convolution (out = in coordinates, stride 1, odd kernel: offsets t and -t at k
    and K-1-k) with no stored kernel map: every GEMM looks its neighbours up in ``index``.

    Forward and, when the map is its own transpose (unique coordinates inside the box), the input
    gradient run ``st_subm_fly_gemm`` (the latter with the offsets' weight slices reversed), both
    over ``order`` (the rows sorted by offset mask; a row of the transposed map has the reversed
    mask, so rows that share one share the other) when given; the weight gradient -- and the input
    gradient otherwise -- take a map queried from the index that lives only for the backward
    call."""

    @staticmethod
    def forward(ctx, features, weights, index: BrickIndex, kernel_offsets, order=None):
        _lib.require_device(features, "features")
        K, C_in, C_out = weights.shape
        assert C_in == features.shape[1], f"weights C_in ({C_in}) != features C_in ({features.shape[1]})"
        assert kernel_offsets.shape[0] == K, "kernel_offsets rows must equal the kernel volume"
        assert features.shape[0] == index.n, "features rows must equal the indexed coordinates"
        features = features.contiguous()
        offs = kernel_offsets.to(torch.int32).contiguous()
        wt = weight_prep(weights.to(features.dtype).contiguous(), _lib.W_TRANSPOSE)
        out = subm_fly_gemm(features, index, offs, wt, order)
        ctx.save_for_backward(features, weights, offs)
        ctx.index, ctx.order = index, order
        return out

    @staticmethod
    def backward(ctx, grad_output):
        features, weights, offs = ctx.saved_tensors
        index = ctx.index
        K = weights.shape[0]
        grad_output = grad_output.to(features.dtype).contiguous()
        grad_input = grad_weights = None
        maps = []  # queried once from the index, held until this function returns

        def queried() -> KernelMap:
            if not maps:
                maps.append(index.query(offs))
            return maps[0]

        if (ctx.needs_input_grad[0] and ctx.needs_input_grad[1] and index.transposable() and
                _concurrent_backward(features, weights.shape[2], index.n)):
            # the weight gradient on a second stream beside the input gradient (its map, pair list and
            # buffers allocated on this stream first; this stream waits for it before returning)
            kmap = queried()
            pl = kmap.pair_list(with_tiles=False)
            bufs = wgrad_buffers(features, grad_output, pl, K, weights.dtype)
            main = torch.cuda.current_stream(features.device)
            side = _side_stream(features.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                grad_weights = wgrad(features, grad_output, kmap, weights.dtype, pairs=pl, buffers=bufs)
            w = weights.to(features.dtype).contiguous()
            grad_input = subm_fly_gemm(grad_output, index, offs, w, ctx.order, reverse_k=True)
            main.wait_stream(side)
            return (grad_input, grad_weights) + (None,) * (len(ctx.needs_input_grad) - 2)
        if ctx.needs_input_grad[0]:
            w = weights.to(features.dtype).contiguous()
            if index.transposable():
                grad_input = subm_fly_gemm(grad_output, index, offs, w, ctx.order, reverse_k=True)
            else:
                n = index.n
                kmap = KernelMap(queried().nbr, n, n, K)
                kmap.set_row_representatives(row_representatives(index.coords))  # repeated coordinates
                kmap.ensure_inverse()
                grad_input = gather_gemm(kmap.fold_output_rows(grad_output), kmap.invnbr, n, 1, kmap.in_masks, w,
                                         n, K)
        if ctx.needs_input_grad[1]:
            kmap = queried()
            grad_weights = wgrad(features, grad_output, kmap, weights.dtype, pairs=kmap.pair_list(with_tiles=False))
        # (index, offsets and, when given, the tile order take no gradient)
        return (grad_input, grad_weights) + (None,) * (len(ctx.needs_input_grad) - 2)
