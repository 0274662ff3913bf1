"""``sparse_conv3d``: the sparse-convolution entry point.

Same signature, argument rules and results as the reference
(``sparsetriton/nn/functional/conv/conv.py:77-239``):

* cubic kernel, uniform stride / dilation / padding (``AssertionError`` otherwise);
* submanifold forces padding ``(k-1)*d//2`` and excludes ``transposed``;
* ``weight`` is (k^3, C_in, C_out); ``bias`` is added to the GEMM's output (fused into its store on
  the precomputed path);
* the coordinate hash table and, per geometry
  ``(k, s, p, d, submanifold, transposed)``, the output coordinates and kernel
  map are cached on the input's ``TensorCache``; a submanifold result shares
  that cache, so a stack of submanifold layers builds its map once;
* ``get_conv_algo()`` picks ``PrecomputedNeighborGEMM`` (kernel map + gather
  GEMM) or ``ImplicitHashFlyGEMM`` (table probes inside the GEMM).

Everything on the path runs as HIP kernels from ``libsparsetriton_amd.so``.
"""

from typing import Tuple, Union

import torch

from sparsetriton_amd import _lib
from sparsetriton_amd.config import ConvAlgo, MIN_TABLE_FACTOR, get_conv_algo, get_h_table_f
from sparsetriton_amd.tensor import SparseTensor
from sparsetriton_amd.utils.hash import HashTable

from .funcs.implicit_hashfly_gemm import (ConvHashOnTheFlyImplicitGEMM, ConvSubmFlyGEMM, InputGradLookup, fly_tile_order,
                                          subm_fly_ok)
from .funcs.implicit_precomputed_gemm import ConvPrecomputedNeighborGEMM, conv_forward_epilogue
from .kmap import (BrickIndex, KernelMap, _target_offsets, brick_out_coords_and_map, build_out_coords_and_map,
                   query_kernel_map, subm_kernel_map)

__all__ = ["sparse_conv3d", "compute_neighbor_indices", "table_capacity"]


def table_capacity(n: int) -> int:
    """Slots for a table of n keys: factor * n with the factor at least 2 (load <= 0.5)."""
    return max(int(n * max(get_h_table_f(), MIN_TABLE_FACTOR)), 16)


def compute_neighbor_indices(
    in_hash_table: HashTable,
    out_coords: torch.Tensor,
    kernel_offsets: torch.Tensor,
    spatial_shape: Tuple[int, int, int],
    stride: int,
    padding: int = 0,
    dilation: int = 1,
) -> torch.Tensor:
    """(N_out, K) int32: row of ``out * stride - kernel_offsets[k]`` if in [0, shape) and present, else -1.

    Same result as the reference (``conv.py:12-75``), computed by one HIP
    kernel (``st_kmap_query``) without materialising the (N_out, K, 4)
    candidate coordinates.  The returned tensor is an (N_out, K) view of the
    offset-major (K, N_out) map.
    """
    kmap = query_kernel_map(in_hash_table, out_coords, kernel_offsets, spatial_shape, stride, n_in=0)
    return kmap.neighbor_indices


def _input_table(tensor: SparseTensor, scale: int) -> HashTable:
    """The coordinate table of ``tensor`` (coordinates * scale for transposed convs), cached.  Its
    clear and insert run when a kernel first reads it (a submanifold precomputed map never does)."""
    cache = tensor._cache
    if scale == 1:
        if cache.hashtable is None:
            t = HashTable(table_capacity(tensor.C.shape[0]), device=tensor.F.device)
            t.insert(tensor.C)
            cache.hashtable = t
        return cache.hashtable
    key = ("scaled_table", scale)
    if key not in cache.kmaps:
        t = HashTable(table_capacity(tensor.C.shape[0]), device=tensor.F.device)
        t.insert(tensor.C, scale=scale)
        cache.kmaps[key] = t
    return cache.kmaps[key]


def _uniform(v, what: str) -> int:
    if isinstance(v, (tuple, list)):
        assert v[0] == v[1] == v[2], f"Only uniform {what} supported for now"
        return int(v[0])
    return int(v)


def sparse_conv3d(
    tensor: SparseTensor,
    weight: torch.Tensor,
    kernel_size: Union[int, Tuple[int, int, int]],
    bias: torch.Tensor = None,
    stride: Union[int, Tuple[int, int, int]] = 1,
    dilation: Union[int, Tuple[int, int, int]] = 1,
    padding: Union[int, Tuple[int, int, int]] = 0,
    transposed: bool = False,
    submanifold: bool = True,
) -> SparseTensor:
    """3-D sparse convolution of ``tensor`` with ``weight`` (k^3, C_in, C_out)."""
    return _sparse_conv3d(tensor, weight, kernel_size, bias, stride, dilation, padding, transposed, submanifold)


def sparse_conv3d_fused(
    tensor: SparseTensor,
    weight: torch.Tensor,
    kernel_size: Union[int, Tuple[int, int, int]],
    bias: torch.Tensor = None,
    stride: Union[int, Tuple[int, int, int]] = 1,
    dilation: Union[int, Tuple[int, int, int]] = 1,
    padding: Union[int, Tuple[int, int, int]] = 0,
    transposed: bool = False,
    submanifold: bool = True,
    scale: torch.Tensor = None,
    shift: torch.Tensor = None,
    residual: torch.Tensor = None,
    relu: bool = False,
) -> SparseTensor:
    """Inference convolution with ``act((conv + bias) * scale + shift + residual)`` applied as the
    GEMM stores its rows (an evaluation-mode conv / batch norm / ReLU block in one pass).  Needs the
    precomputed-map algorithm and no autograd."""
    if get_conv_algo() != ConvAlgo.PrecomputedNeighborGEMM:
        raise ValueError("the fused epilogue runs on the precomputed-map algorithm")
    if torch.is_grad_enabled() and (tensor.F.requires_grad or weight.requires_grad or
                                    (bias is not None and bias.requires_grad)):
        raise ValueError("the fused epilogue is an inference path (no autograd); call it under torch.no_grad()")
    return _sparse_conv3d(tensor, weight, kernel_size, bias, stride, dilation, padding, transposed, submanifold,
                          epilogue=(scale, shift, residual, relu))


def _sparse_conv3d(tensor, weight, kernel_size, bias, stride, dilation, padding, transposed, submanifold,
                   epilogue=None) -> SparseTensor:
    if isinstance(kernel_size, (tuple, list)):
        assert kernel_size[0] == kernel_size[1] == kernel_size[2], "Only cubic kernels supported for now"
    k = _uniform(kernel_size, "kernel")
    s = _uniform(stride, "stride")
    d = _uniform(dilation, "dilation")
    if submanifold:
        padding = ((k - 1) * d) // 2
    p = _uniform(padding, "padding")
    if submanifold:
        assert not transposed, "Submanifold convolution does not support transposed=True"

    device = tensor.F.device
    K, C_in, C_out = weight.shape
    assert C_in == tensor.F.shape[1], f"Input channels in weight({C_in}) and tensor({tensor.F.shape[1]}) must match"
    assert K == k ** 3, f"Kernel size in weight({K}) and argument({k ** 3}) must match"
    _lib.require_device(tensor.F, "SparseTensor features")

    scale = s if (transposed and s > 1) else 1
    lookup_shape = tuple(int(v) * scale for v in tensor.spatial_shape)
    subm_fast = submanifold and s == 1 and ((k - 1) * d) // 2 == p
    cache_key = (k, s, p, d, submanifold, transposed)
    algo = get_conv_algo()

    # A fresh map build ends with an asynchronous copy of the table's status words; once the
    # forward is queued the host waits for that copy (not for the forward) and raises if a
    # coordinate could not be keyed or the table overflowed -- rows the map would silently lack.
    table_status = None
    in_table = None
    if algo == ConvAlgo.PrecomputedNeighborGEMM:
        hit = tensor._cache.neighbor_indices.get(cache_key)
        if hit is not None:
            out_coords, kmap, new_shape = hit
        else:
            built = None
            if subm_fast:
                out_coords, new_shape = tensor.C, tensor.spatial_shape
                offsets = _target_offsets(k, d, p, False, device)
                # brick index + query in one launch; the symmetric claim is checked against its
                # duplicate / out-of-bounds counts
                built = subm_kernel_map(tensor.C, tensor.batch_size, tensor.spatial_shape, offsets,
                                        symmetric=(k % 2 == 1))
                if built is not None:
                    kmap, table_status = built
                else:
                    in_table = _input_table(tensor, scale)
                    kmap = query_kernel_map(in_table, tensor.C, offsets, tensor.spatial_shape, 1,
                                            tensor.C.shape[0], symmetric=(k % 2 == 1))
            else:
                # brick indexes of the candidates and of the inputs; the hash tables when a box cannot
                # be indexed or a row's batch index lies outside the tensor's batch count
                built = brick_out_coords_and_map(tensor.C, tensor.batch_size, tensor.spatial_shape, k, s, d, p,
                                                 transposed)
                if built is not None:
                    out_coords, new_shape, _, kmap, table_status = built
                else:
                    in_table = _input_table(tensor, scale)
                    out_coords, new_shape, _, kmap, _ = build_out_coords_and_map(
                        tensor.C, tensor.spatial_shape, k, s, d, p, transposed, in_table=in_table, with_map=True)
            if built is None:
                table_status = in_table.snapshot()
            tensor._cache.neighbor_indices[cache_key] = (out_coords, kmap, new_shape)
        if out_coords.shape[0] == 0:
            _raise_table_errors(table_status, in_table)
            return _empty(tensor, C_out, new_shape)
        if hit is None and torch.is_grad_enabled() and (tensor.F.requires_grad or weight.requires_grad):
            # the weight gradient's pair list is built with the tile plan, alongside it
            kmap.forward_tiles(with_pairs=True)
        if epilogue is not None:
            out_feats = conv_forward_epilogue(tensor.F, weight, kmap, bias, *epilogue)
        else:
            out_feats = ConvPrecomputedNeighborGEMM.apply(tensor.F, weight, kmap, bias)
    elif algo == ConvAlgo.ImplicitHashFlyGEMM and _brick_index(tensor, subm_fast and k % 2 == 1, K, C_in, C_out):
        # submanifold, odd kernel, built shape: lookups in the coordinates' brick index inside the GEMM
        index = _brick_index(tensor, True, K, C_in, C_out)
        table_status = index.status
        out_coords, new_shape = tensor.C, tensor.spatial_shape
        if out_coords.shape[0] == 0:
            _raise_table_errors(table_status, None)
            return _empty(tensor, C_out, new_shape)
        offsets = _target_offsets(k, d, p, False, device)
        order = fly_tile_order(index, offsets, (k, d, p))
        out_feats = ConvSubmFlyGEMM.apply(tensor.F, weight, index, offsets, order)
        if bias is not None:
            out_feats = out_feats + bias.to(out_feats.dtype)  # as the hash-probing branch below
    elif algo == ConvAlgo.ImplicitHashFlyGEMM:
        hkey = ("hashfly",) + cache_key
        hit = tensor._cache.kmaps.get(hkey)
        in_table = _input_table(tensor, scale)
        in_keys, in_vals = in_table.table_keys, in_table.table_values  # runs a deferred insert
        if hit is None:
            if subm_fast:
                out_coords, new_shape = tensor.C, tensor.spatial_shape
                offsets = _target_offsets(k, d, p, False, device).to(tensor.C.dtype)
                table_status = in_table.snapshot()
                gl = InputGradLookup(in_keys, in_vals, 1, 1, new_shape, tensor.spatial_shape,
                                     duplicate_check=table_status)
            else:
                out_coords, new_shape, offsets, _, out_table = build_out_coords_and_map(
                    tensor.C, tensor.spatial_shape, k, s, d, p, transposed, in_table=in_table, with_map=False)
                mul, div = (s, 1) if transposed else (1, s)
                table_status = in_table.snapshot()
                gl = InputGradLookup(out_table.table_keys, out_table.table_values, mul, div, new_shape,
                                     tensor.spatial_shape, duplicate_check=table_status)
            hit = (out_coords, new_shape, offsets, gl)
            tensor._cache.kmaps[hkey] = hit
        out_coords, new_shape, offsets, gl = hit
        if out_coords.shape[0] == 0:
            _raise_table_errors(table_status, in_table)
            return _empty(tensor, C_out, new_shape)
        out_feats = ConvHashOnTheFlyImplicitGEMM.apply(
            tensor.F, weight, out_coords, offsets, in_keys, in_vals, lookup_shape,
            1 if transposed else s, tensor.C, gl)
        if bias is not None:
            # in the features' dtype, as the reference's in-place `out_feats += bias` (conv.py:227-228);
            # the precomputed path adds it inside the GEMM's store instead
            out_feats = out_feats + bias.to(out_feats.dtype)
    else:
        raise ValueError(f"unknown convolution algorithm {algo}")
    _raise_table_errors(table_status, in_table)

    if submanifold and (out_coords is tensor.C or (out_coords.shape == tensor.C.shape
                                                   and torch.equal(out_coords, tensor.C))):
        return tensor.replace(out_feats)
    return SparseTensor(feats=out_feats, coords=out_coords, spatial_shape=new_shape, batch_size=tensor.batch_size)


def _brick_index(tensor: SparseTensor, eligible: bool, K: int, C_in: int, C_out: int):
    """The tensor's cached brick index when the hash-fly algorithm can look a submanifold
    convolution's neighbours up in it (``st_subm_fly_gemm`` built for the shape, box indexable),
    else None.  The index depends on the coordinates only, so every layer over them shares it."""
    if not eligible or tensor.C.dtype not in (torch.int16, torch.int32) or \
            not subm_fly_ok(int(tensor.F.shape[0]), C_in, C_out, K, tensor.F.dtype):
        return None
    key = ("brick_index", int(tensor.batch_size), tuple(int(v) for v in tensor.spatial_shape))
    if key not in tensor._cache.kmaps:
        tensor._cache.kmaps[key] = BrickIndex.build(tensor.C, tensor.batch_size, tensor.spatial_shape)
    return tensor._cache.kmaps[key]


def _raise_table_errors(status, table) -> None:
    if status is not None:
        status.raise_errors(table.capacity if table is not None else 0)


def _empty(tensor: SparseTensor, C_out: int, new_shape) -> SparseTensor:
    device = tensor.F.device
    return SparseTensor(
        feats=torch.empty((0, C_out), device=device, dtype=tensor.F.dtype),
        coords=torch.empty((0, 4), device=device, dtype=tensor.C.dtype),
        spatial_shape=new_shape,
        batch_size=tensor.batch_size,
    )
