"""Gather-GEMM sparse convolution over a precomputed kernel map (HIP/MFMA).

``ConvPrecomputedNeighborGEMM.apply(features, weights, neighbor_indices)`` has
the reference's signature and meaning
(``sparsetriton/nn/functional/conv/funcs/implicit_precomputed_gemm.py:233-324``):

    out[o] = sum_k features[nbr[o, k]] @ weights[k]      (nbr = -1 contributes 0)

with ``features`` (N_in, C_in), ``weights`` (K, C_in, C_out), output in the
features' dtype, fp32 accumulation.  ``neighbor_indices`` is either the
reference's (N_out, K) int32 tensor (any strides) or a ``KernelMap`` built by
this package (which also carries row masks and the transposed map).

Kernels (``libsparsetriton_amd.so``):
  forward   st_gather_gemm with rows tiled in mask-sorted order, weights
            re-laid (K, C_out, C_in);
  dgrad     st_gather_gemm over the transposed map (also mask-sorted), weights
            as stored -- a gather, so no atomics and a deterministic result.
            An odd-kernel submanifold map is its own transpose with offsets
            reversed, so dgrad gathers through the forward map, masks and tile
            order with the weights reversed along k (no inverse map is built);
  wgrad     st_wgrad_pairs over the (offset, out)-sorted pair list in
            equal-size chunks, fixed-order reduce; for 16-bit rows with 128-multiple
            channel counts over a dense map, st_wgrad over the map itself (windows of
            output rows, four offsets a workgroup sharing each staged dY row).
"""

import os
from typing import Optional

import torch

from sparsetriton_amd import _lib
from sparsetriton_amd.nn.functional.conv.kmap import KernelMap

__all__ = ["ConvPrecomputedNeighborGEMM", "wgrad_splits"]


def wgrad_splits(n_rows: int) -> int:
    """Row splits per offset for the weight gradient: ~16k map rows per workgroup."""
    return max(1, min(4096, (n_rows + 16383) // 16384))


def _as_kmap(neighbor_indices, n_in: int) -> KernelMap:
    if isinstance(neighbor_indices, KernelMap):
        return neighbor_indices
    return KernelMap.from_neighbor_indices(neighbor_indices, n_in)


def gather_gemm(A: torch.Tensor, map_t: torch.Tensor, k_stride: int, r_stride: int, masks, Bt: torch.Tensor,
                n_dst: int, K: int, rows=None, bias=None) -> torch.Tensor:
    """out[rows[r]] = sum_k A[map[k, r]] @ Bt[k]^T (+ bias) on the GPU (rows = identity when None)."""
    Kd = A.shape[1]
    Nd = Bt.shape[1]
    out = torch.empty((n_dst, Nd), dtype=A.dtype, device=A.device)
    W = (K + 31) // 32
    _lib.call("st_gather_gemm", _lib.ptr(A), A.shape[0], _lib.ptr(map_t), k_stride, r_stride,
              _lib.ptr(masks), W, _lib.ptr(rows), _lib.ptr(Bt), _lib.ptr(bias), _lib.ptr(out), n_dst, K, Kd, Nd,
              _lib.compute_code(A.dtype), _lib.stream_of(A.device))
    return out


def tiled_ok(dtype: torch.dtype, Kd: int) -> bool:
    """Whether st_gather_gemm_tiled covers this reduction width (it covers every common one)."""
    return Kd <= (64 if _lib.compute_code(dtype) == 0 else 128)


def gather_gemm_tiled(A: torch.Tensor, tiles, Bt: torch.Tensor, n_dst: int, K: int, bias=None,
                      reverse_k: bool = False) -> torch.Tensor:
    """out[perm[t]] = sum over the tile's offsets of A[source] @ Bt[k]^T (+ bias), over a tile plan;
    with ``reverse_k`` offset k's sources meet Bt[K - 1 - k]."""
    Kd = A.shape[1]
    Nd = Bt.shape[1]
    out = torch.empty((n_dst, Nd), dtype=A.dtype, device=A.device)
    _lib.call("st_gather_gemm_tiled", _lib.ptr(A), A.shape[0], tiles.perm_ptr, tiles.nk_ptr,
              tiles.klist_ptr, tiles.tmap_ptr, _lib.ptr(Bt), _lib.ptr(bias), _lib.ptr(out), n_dst, K,
              Kd, Nd, _lib.compute_code(A.dtype), _lib.GATHER_REVERSE_K if reverse_k else 0,
              _lib.stream_of(A.device))
    return out


def gather_gemm_fwd(A: torch.Tensor, kmap: KernelMap, Bt: torch.Tensor, bias=None) -> torch.Tensor:
    """Forward: out rows in the mask-sorted order of the forward plan, over its tile plan; ``bias``
    (C_out, A's dtype) is added as the rows are stored."""
    if tiled_ok(A.dtype, A.shape[1]):
        return gather_gemm_tiled(A, kmap.forward_tiles(), Bt, kmap.n_out, kmap.K, bias=bias)
    plan = kmap.forward_plan()
    return gather_gemm(A, kmap.nbr, kmap.k_stride, kmap.r_stride, kmap.out_masks, Bt, kmap.n_out, kmap.K,
                       rows=plan.perm, bias=bias)


def conv_forward_epilogue(features: torch.Tensor, weights: torch.Tensor, kmap: KernelMap, bias, scale, shift,
                          residual, relu: bool) -> torch.Tensor:
    """Forward with the store epilogue ``act((sum + bias) * scale + shift + residual)`` (inference:
    no autograd).  ``scale`` / ``shift`` fp32 (C_out) or None; ``bias`` and ``residual`` (N_out, C_out)
    in the features' dtype, residual rows in output order."""
    _lib.require_device(features, "features")
    N_in, C_in = features.shape
    K, C_in_w, C_out = weights.shape
    assert C_in_w == C_in, f"weights C_in ({C_in_w}) != features C_in ({C_in})"
    assert kmap.K == K, f"kernel map has {kmap.K} offsets, weights {K}"
    if not tiled_ok(features.dtype, C_in):
        raise ValueError(f"the fused-epilogue forward covers reduction widths up to the tiled kernels' ({C_in})")
    A = features.contiguous()
    wt = weight_prep(weights.to(A.dtype).contiguous(), _lib.W_TRANSPOSE)
    b = None if bias is None else bias.detach().to(A.dtype).contiguous()
    sc = None if scale is None else scale.detach().to(torch.float32).contiguous()
    sh = None if shift is None else shift.detach().to(torch.float32).contiguous()
    res = None
    if residual is not None:
        assert residual.shape == (kmap.n_out, C_out), "residual must be (N_out, C_out)"
        res = residual.detach().to(A.dtype).contiguous()
    tiles = kmap.forward_tiles()
    out = torch.empty((kmap.n_out, C_out), dtype=A.dtype, device=A.device)
    _lib.call("st_gather_gemm_tiled_epilogue", _lib.ptr(A), N_in, tiles.perm_ptr, tiles.nk_ptr,
              tiles.klist_ptr, tiles.tmap_ptr, _lib.ptr(wt), _lib.ptr(b), _lib.ptr(sc), _lib.ptr(sh),
              _lib.ptr(res), int(bool(relu)), _lib.ptr(out), kmap.n_out, K, C_in, C_out,
              _lib.compute_code(A.dtype), _lib.stream_of(A.device))
    return out


def gather_gemm_dgrad(dY: torch.Tensor, kmap: KernelMap, W: torch.Tensor) -> torch.Tensor:
    """Input gradient over the transposed map, in the mask-sorted order of the backward plan.

    For a symmetric (odd-kernel submanifold) map the transpose is the map read
    with offsets reversed: dX[i] = sum_j dY[nbr[j, i]] @ W[K-1-j]^T; the tiled GEMM
    takes the reversal as it addresses the weights (no reversed copy)."""
    symmetric = kmap.symmetric  # (first: resolving it also finds repeated output rows, which the fold needs)
    dY = kmap.fold_output_rows(dY)
    if tiled_ok(dY.dtype, dY.shape[1]):
        return gather_gemm_tiled(dY, kmap.backward_tiles(), W, kmap.n_in, kmap.K, reverse_k=symmetric)
    if symmetric:
        W = weight_prep(W, _lib.W_REVERSE)
    plan = kmap.backward_plan()
    if kmap.symmetric:
        return gather_gemm(dY, kmap.nbr, kmap.k_stride, kmap.r_stride, kmap.out_masks, W, kmap.n_in, kmap.K,
                           rows=plan.perm)
    return gather_gemm(dY, kmap.invnbr, kmap.n_in, 1, kmap.in_masks, W, kmap.n_in, kmap.K, rows=plan.perm)


def weight_prep(weights: torch.Tensor, mode: int) -> torch.Tensor:
    K, C_in, C_out = weights.shape
    shape = (K, C_out, C_in) if mode == _lib.W_TRANSPOSE else (K, C_in, C_out)
    out = torch.empty(shape, dtype=weights.dtype, device=weights.device)
    _lib.call("st_weight_prep", _lib.ptr(weights), _lib.ptr(out), K, C_in, C_out, mode,
              _lib.feat_code(weights.dtype), _lib.stream_of(weights.device))
    return out


def column_sum(Y: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """Sum over the rows of Y (n, C) with fp32 accumulation, in a fixed order (the bias gradient)."""
    n, C = Y.shape
    partials = torch.empty((1024 * C,), dtype=torch.float32, device=Y.device)
    out = torch.empty((C,), dtype=out_dtype, device=Y.device)
    _lib.call("st_column_sum", _lib.ptr(Y), n, C, _lib.feat_code(Y.dtype), _lib.ptr(partials), _lib.ptr(out),
              _lib.feat_code(out_dtype), _lib.stream_of(Y.device))
    return out


def wgrad_buffers(X: torch.Tensor, dY: torch.Tensor, pl, K: int, dw_dtype: torch.dtype):
    """(partials, dW) for ``wgrad`` over the pair list ``pl``."""
    C_in, C_out = X.shape[1], dY.shape[1]
    partials = torch.empty((max(pl.max_chunks, 1) * C_in * C_out,), dtype=torch.float32, device=X.device)
    return partials, torch.empty((K, C_in, C_out), dtype=dw_dtype, device=X.device)


def wgrad(X: torch.Tensor, dY: torch.Tensor, kmap: KernelMap, dw_dtype: torch.dtype, pairs=None,
          buffers=None) -> torch.Tensor:
    """dW[k] = sum over pairs (i, o) of offset k of X[i]^T dY[o], over the map's pair list (or
    ``pairs``, a PairList of it); ``buffers`` from ``wgrad_buffers`` (else allocated here)."""
    K, C_in, C_out = kmap.K, X.shape[1], dY.shape[1]
    pl = kmap.pair_list() if pairs is None else pairs
    partials, dW = wgrad_buffers(X, dY, pl, K, dw_dtype) if buffers is None else buffers
    _lib.call("st_wgrad_pairs", _lib.ptr(X), X.shape[0], _lib.ptr(dY), dY.shape[0], pl.pairs_ptr,
              pl.kstart_ptr, pl.cstart_ptr, K, pl.chunk, pl.max_chunks, pl.corder_ptr, C_in, C_out,
              _lib.compute_code(X.dtype),
              _lib.ptr(partials), _lib.ptr(dW), _lib.feat_code(dw_dtype), _lib.stream_of(X.device))
    return dW


def window_splits(n_out: int, K: int, C_in: int, C_out: int) -> int:
    """Output-row windows per offset for st_wgrad's window kernel (16-bit rows, C_in and C_out
    multiples of 128): a workgroup per (window, 128 x 128 channel tile, pair of offsets), one
    round of 512 workgroups (two per CU), windows of at least 1024 rows.
    ST_WGRAD_WINDOW_ROUNDS=r asks for r rounds."""
    items = (C_in // 128) * (C_out // 128) * ((K + 1) // 2)
    rounds = max(1, int(os.environ.get("ST_WGRAD_WINDOW_ROUNDS", "1")))
    return max(1, min((n_out + 1023) // 1024, max(1, (512 * rounds) // items)))


def window_slab() -> int:
    """Slab (rows) of ``KernelMap.window_order`` for the window weight gradient; 0 takes the map's
    columns in their own order (ST_WGRAD_SLAB)."""
    return int(os.environ.get("ST_WGRAD_SLAB", "4096"))


def window_wgrad_ok(X: torch.Tensor, dY: torch.Tensor, kmap: KernelMap) -> bool:
    """Whether the weight gradient runs over the map itself (st_wgrad's window kernel, the map's
    columns in ``window_order``) instead of the pair list: only when ST_WGRAD_PATH=window asks
    for it, for 16-bit rows with C_in and C_out multiples of 128.  On config 5 (1 M rows, 18
    pairs a row) it moves half the fabric bytes of the pair-list kernel (2.6 vs 5.2 GB) at the
    same time (1.05 vs 1.04 ms), so the pair list stays the default."""
    if os.environ.get("ST_WGRAD_PATH", "pairs") != "window":
        return False
    return X.dtype in (torch.bfloat16, torch.float16) and X.shape[1] % 128 == 0 and dY.shape[1] % 128 == 0


def scan_splits(X: torch.Tensor, dY: torch.Tensor, n_out: int, K: int) -> int:
    """Row splits per offset for ``wgrad_scan``: ``window_splits`` where st_wgrad takes the window
    kernel, else ``wgrad_splits``."""
    C_in, C_out = X.shape[1], dY.shape[1]
    if X.dtype in (torch.bfloat16, torch.float16) and C_in % 128 == 0 and C_out % 128 == 0:
        return window_splits(n_out, K, C_in, C_out)
    return wgrad_splits(n_out)


def scan_buffers(X: torch.Tensor, dY: torch.Tensor, K: int, splits: int, dw_dtype: torch.dtype):
    """(partials, dW) for ``wgrad_scan`` with ``splits`` row splits."""
    C_in, C_out = X.shape[1], dY.shape[1]
    return (torch.empty((K * splits * C_in * C_out,), dtype=torch.float32, device=X.device),
            torch.empty((K, C_in, C_out), dtype=dw_dtype, device=X.device))


def wgrad_scan(X: torch.Tensor, dY: torch.Tensor, kmap: KernelMap, dw_dtype: torch.dtype,
               splits: Optional[int] = None, buffers=None, order=None) -> torch.Tensor:
    """Weight gradient over the map itself, no pair list (st_wgrad): for 16-bit rows with C_in and
    C_out multiples of 128 the window kernel (over the map's columns in the order ``order`` =
    ``KernelMap.window_order(slab)`` when given), else map columns compacted on the fly;
    ``splits`` from ``scan_splits`` and ``buffers`` from ``scan_buffers`` unless given."""
    K, C_in, C_out = kmap.K, X.shape[1], dY.shape[1]
    if splits is None:
        splits = scan_splits(X, dY, kmap.n_out, K)
    partials, dW = scan_buffers(X, dY, K, splits, dw_dtype) if buffers is None else buffers
    if order is None:
        m, ks, rs, rows = kmap.nbr, kmap.k_stride, kmap.r_stride, None
    else:
        rows, m = order
        ks, rs = kmap.n_out, 1
    _lib.call("st_wgrad", _lib.ptr(X), X.shape[0], _lib.ptr(dY), _lib.ptr(m), ks, rs,
              None if rows is None else _lib.ptr(rows), kmap.n_out,
              K, C_in, C_out, _lib.feat_code(X.dtype), _lib.ptr(partials), splits, _lib.ptr(dW),
              _lib.feat_code(dw_dtype), _lib.stream_of(X.device))
    return dW


def window_order(kmap: KernelMap):
    slab = window_slab()
    return kmap.window_order(slab) if slab > 0 else None


def weight_gradient(X: torch.Tensor, dY: torch.Tensor, kmap: KernelMap, dw_dtype: torch.dtype) -> torch.Tensor:
    """dW by the path the backward takes: the window kernel over the map where
    ``window_wgrad_ok``, else the pair list."""
    if window_wgrad_ok(X, dY, kmap):
        return wgrad_scan(X, dY, kmap, dw_dtype, order=window_order(kmap))
    return wgrad(X, dY, kmap, dw_dtype)


_SIDE_STREAMS = {}


def _side_stream(device: torch.device) -> "torch.cuda.Stream":
    """One extra stream per device (default priority) for the weight gradient."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _SIDE_STREAMS:
        _SIDE_STREAMS[idx] = torch.cuda.Stream(device=idx)
    return _SIDE_STREAMS[idx]


def _concurrent_backward(X: torch.Tensor, C_out: int, n_rows: int) -> bool:
    """Whether the weight gradient runs beside the input gradient.  At 16-bit 128 x 128 both run
    one workgroup per CU (the two-tile wide gather, the 128 x 128 per-wave weight gradient), which
    leaves issue slots the other kernel fills: config 5 step 2.65 -> 2.53 ms.  Elsewhere the kernels
    already fill the CUs and the cross-stream waits cost more than the overlap gains (config 2 bf16
    0.186 -> 0.21 ms, config 3 / 4 3-8 % slower).  ST_CONCURRENT_BACKWARD=0 / 2 forces it off / on."""
    mode = os.environ.get("ST_CONCURRENT_BACKWARD", "1")
    if mode in ("0", "2"):
        return mode == "2"
    return (X.dtype in (torch.bfloat16, torch.float16) and X.shape[1] % 128 == 0 and C_out % 128 == 0 and
            n_rows >= 1 << 18)


class ConvPrecomputedNeighborGEMM(torch.autograd.Function):
    """Sparse convolution with a precomputed neighbour map (gather-GEMM on MFMA)."""

    @staticmethod
    def forward(ctx, features, weights, neighbor_indices, bias=None):
        """The reference's three arguments, plus an optional ``bias`` (C_out) added in the GEMM's
        store (the reference adds it afterwards, ``conv.py:227-228``)."""
        _lib.require_device(features, "features")
        N_in, C_in = features.shape
        K, C_in_w, C_out = weights.shape
        assert C_in_w == C_in, f"weights C_in ({C_in_w}) != features C_in ({C_in})"
        kmap = _as_kmap(neighbor_indices, N_in)
        assert kmap.K == K, f"kernel map has {kmap.K} offsets, weights {K}"
        features = features.contiguous()
        w = weights.to(features.dtype).contiguous()
        wt = weight_prep(w, _lib.W_TRANSPOSE)
        b = None
        if bias is not None:
            assert bias.shape == (C_out,), f"bias must have shape ({C_out},), got {tuple(bias.shape)}"
            b = bias.to(features.dtype).contiguous()
        out = gather_gemm_fwd(features, kmap, wt, bias=b)
        ctx.save_for_backward(features, weights)
        ctx.kmap = kmap
        ctx.bias_dtype = None if bias is None else bias.dtype
        return out

    @staticmethod
    def backward(ctx, grad_output):
        features, weights = ctx.saved_tensors
        kmap = ctx.kmap
        grad_output = grad_output.to(features.dtype).contiguous()
        grad_input = grad_weights = None
        if (ctx.needs_input_grad[0] and ctx.needs_input_grad[1] and
                _concurrent_backward(features, weights.shape[2], min(kmap.n_in, kmap.n_out))):
            # The two gradients are independent: the weight gradient runs on a second stream beside
            # the input gradient (every buffer it touches is allocated on this stream first, and this
            # stream waits for it before returning).
            if window_wgrad_ok(features, grad_output, kmap):
                splits = scan_splits(features, grad_output, kmap.n_out, kmap.K)
                bufs = scan_buffers(features, grad_output, kmap.K, splits, weights.dtype)
                order = window_order(kmap)
                run = lambda: wgrad_scan(features, grad_output, kmap, weights.dtype, splits, bufs, order)  # noqa: E731
            else:
                pl = kmap.pair_list()
                bufs = wgrad_buffers(features, grad_output, pl, kmap.K, weights.dtype)
                run = lambda: wgrad(features, grad_output, kmap, weights.dtype, pairs=pl, buffers=bufs)  # noqa: E731
            main = torch.cuda.current_stream(features.device)
            side = _side_stream(features.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                grad_weights = run()
            w = weights.to(features.dtype).contiguous()
            grad_input = gather_gemm_dgrad(grad_output, kmap, w)
            main.wait_stream(side)
        else:
            if ctx.needs_input_grad[0]:
                w = weights.to(features.dtype).contiguous()
                # dX[i] = sum_k dY[invnbr[k, i]] @ W[k]^T: W[k] (C_in, C_out) is already the (Nd, Kd) operand.
                grad_input = gather_gemm_dgrad(grad_output, kmap, w)
            if ctx.needs_input_grad[1]:
                grad_weights = weight_gradient(features, grad_output, kmap, weights.dtype)
        grad_bias = None
        if ctx.bias_dtype is not None and len(ctx.needs_input_grad) > 3 and ctx.needs_input_grad[3]:
            grad_bias = column_sum(grad_output, ctx.bias_dtype)
        return grad_input, grad_weights, None, grad_bias
