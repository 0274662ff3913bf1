"""Kernel offsets, output coordinates and kernel maps.

Public functions keep the reference's names and meaning
(``sparsetriton/nn/functional/conv/kmap.py:104-495``):

* ``generate_base_offsets`` -- the k^3 offsets ``(i - k//2) * d`` per axis,
  enumerated x-major / z-minor (``torch.meshgrid(indexing="ij")``), so offset
  index ``k = (ix * ks + iy) * ks + iz``.
* ``compute_target_offsets_normal`` / ``_transposed`` -- the per-offset shift
  the neighbour lookup subtracts: input = output * stride - t_k.
* ``build_out_coords`` -- (out_coords, new_spatial_shape, kernel_offsets).

The output coordinates of a strided / transposed convolution come from a brick
index of the candidates' output box (``st_outcoords_brick_*``) and its kernel
map from a query of each output row in the inputs' brick index
(``st_kmap_strided_query``, ``st_outcoords_brick_inverse``); where a box cannot
be indexed, from hash tables (``st_outcoords_plan`` / ``st_outcoords_emit``).
The submanifold map comes from the coordinates' brick index (``st_kmap_subm``),
or the table query (``st_kmap_query``) for boxes too large for it.  Maps are stored
offset-major (K, N) int32 with per-row offset bitmasks, in both directions:
``nbr[k, o]`` is the input row feeding output ``o`` through offset ``k`` and
``invnbr[k, i]`` the output row input ``i`` feeds.  Every kernel that walks rows
then touches each offset's column with coalesced accesses; the reference's
(N, K) layout is exposed as a transposed view.
"""

from typing import Optional, Tuple

import ctypes
import functools
import torch

from sparsetriton_amd import _lib
from sparsetriton_amd.config import get_tile_slab_bits
from sparsetriton_amd.utils.hash import HashTable

__all__ = [
    "generate_base_offsets",
    "compute_target_offsets_normal",
    "compute_target_offsets_transposed",
    "build_out_coords",
    "brick_out_coords_and_map",
    "KernelMap",
    "query_kernel_map",
    "subm_kernel_map",
    "row_representatives",
    "TilePlan",
    "TileMap",
    "PairList",
    "MapPlan",
    "out_spatial_shape",
]


# --------------------------------------------------------------- offsets/shape

def generate_base_offsets(kernel_size, dilation, device) -> torch.Tensor:
    """(k^3, 3) offsets ``(i - k//2) * d``, x-major (``kmap.py:104-132``)."""
    ks = [int(v) for v in (kernel_size.tolist() if isinstance(kernel_size, torch.Tensor) else kernel_size)]
    dil = dilation.to("cpu") if isinstance(dilation, torch.Tensor) else torch.as_tensor(dilation)
    axes = [torch.arange(s) - (s // 2) for s in ks]
    grid = torch.meshgrid(*axes, indexing="ij")
    return (torch.stack(grid, dim=-1).reshape(-1, 3) * dil).to(device)


def compute_target_offsets_normal(base_offsets, padding, dilation, kernel_size) -> torch.Tensor:
    """t_k = -base + p - (k-1)*d//2: input = out*s - t_k (``kmap.py:135-155``)."""
    return -base_offsets + padding - (kernel_size - 1) * dilation // 2


def compute_target_offsets_transposed(base_offsets, padding, dilation, kernel_size, stride=None) -> torch.Tensor:
    """t_k = base - p + (k-1)*d//2: output = in*s + t_k (``kmap.py:158-180``)."""
    return base_offsets - padding + (kernel_size - 1) * dilation // 2


@functools.lru_cache(maxsize=256)
def _target_offsets_on(kernel_size: int, dilation: int, padding: int, transposed: bool,
                       device: torch.device) -> torch.Tensor:
    ks = torch.tensor([kernel_size] * 3)
    dil = torch.tensor([dilation] * 3)
    pad = torch.tensor([padding] * 3)
    base = generate_base_offsets(ks, dil, "cpu")
    if transposed:
        t = compute_target_offsets_transposed(base, pad, dil, ks)
    else:
        t = compute_target_offsets_normal(base, pad, dil, ks)
    return t.to(torch.int32).to(device)


def _target_offsets(kernel_size: int, dilation: int, padding: int, transposed: bool, device) -> torch.Tensor:
    """(K, 3) int32 offsets on ``device``, built once per geometry and device: every map build
    of a layer reuses them (no host-side tensor ops, host-to-device copy or dtype conversion).
    The returned tensor is shared; callers must not modify it."""
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return _target_offsets_on(int(kernel_size), int(dilation), int(padding), bool(transposed), dev)


def out_spatial_shape(spatial_shape, kernel_size: int, stride: int, dilation: int, padding: int,
                      transposed: bool) -> Tuple[int, int, int]:
    """Output grid of a convolution (``kmap.py:254-258`` normal, ``:373-377`` transposed)."""
    k, s, d, p = kernel_size, stride, dilation, padding
    if transposed:
        return tuple((int(v) - 1) * s + (k - 1) * d - 2 * p + 1 for v in spatial_shape)
    return tuple((int(v) - (k - 1) * d + 2 * p - 1) // s + 1 for v in spatial_shape)


def _mask_words(K: int) -> int:
    return (K + 31) // 32


# ------------------------------------------------------------------ KernelMap

class KernelMap:
    """Kernel map of one convolution geometry on one coordinate set.

    ``nbr`` (K, N_out) int32, offset-major, -1 where no neighbour;
    ``out_masks`` (N_out, W) row bitmasks of ``nbr`` (W = ceil(K/32));
    ``invnbr`` (K, N_in) and ``in_masks`` (N_in, W) the transposed map, built
    lazily by ``ensure_inverse`` for the input gradient.
    ``nbr`` may also be a caller's (N_out, K) tensor (``k_stride``/``r_stride``).
    """

    def __init__(self, nbr: torch.Tensor, n_in: int, n_out: int, K: int, out_masks: Optional[torch.Tensor] = None,
                 invnbr: Optional[torch.Tensor] = None, in_masks: Optional[torch.Tensor] = None,
                 k_stride: Optional[int] = None, r_stride: Optional[int] = None, symmetric: bool = False,
                 symmetry_check=None):
        self.nbr = nbr
        # A submanifold map of an odd kernel is its own transpose with the offsets
        # reversed: base_{K-1-k} = -base_k, so nbr[k, o] = i <=> nbr[K-1-k, i] = o --
        # provided the coordinates are unique and inside the query bounds (a row
        # outside them keeps its in-bounds neighbours, but no row finds it).  The
        # input gradient then gathers through ``nbr`` itself, with the forward's
        # masks and tile order and reversed weights.  ``symmetry_check`` (a
        # StatusSnapshot of the query's duplicate / out-of-bounds counts) confirms
        # the claim the first time it is needed; otherwise the transpose is built.
        self._symmetric = bool(symmetric) and int(n_in) == int(n_out)
        self._symmetry_check = symmetry_check if self._symmetric else None
        # Output rows repeating a coordinate have identical map rows: one input then feeds
        # several outputs through one offset, which ``invnbr`` cannot hold.  ``row_rep`` (the
        # lowest row of each output's coordinate, when any repeat) folds them: the transposed
        # map is built over the representatives only and the input gradient first sums dY
        # over each coordinate's rows.  ``_out_coords`` lets the symmetry check find them.
        self.row_rep = None
        self._out_coords = None
        self.raw = False  # a caller's map: its transpose is checked for conflicts
        self._conflicts = None
        self.n_in, self.n_out, self.K = int(n_in), int(n_out), int(K)
        self.k_stride = int(n_out) if k_stride is None else int(k_stride)
        self.r_stride = 1 if r_stride is None else int(r_stride)
        self.out_masks = out_masks
        self.invnbr = invnbr
        self.in_masks = in_masks
        self._fwd = None
        self._bwd = None
        self._fwd_tiles = None
        self._bwd_tiles = None
        self._pairs = {}
        self._window_orders = {}

    @classmethod
    def from_neighbor_indices(cls, neighbor_indices: torch.Tensor, n_in: int) -> "KernelMap":
        """Wrap a caller's (N_out, K) int32 map (any strides) without copying it."""
        assert neighbor_indices.ndim == 2, "neighbor_indices must be (N_out, K)"
        nbr = neighbor_indices
        if nbr.dtype != torch.int32:
            nbr = nbr.to(torch.int32)
        n_out, K = nbr.shape
        km = cls(nbr, n_in, n_out, K, k_stride=nbr.stride(1), r_stride=nbr.stride(0))
        km.raw = True
        return km

    @property
    def symmetric(self) -> bool:
        """Whether ``nbr`` read with offsets reversed is the transposed map (resolved once,
        waiting at most for the map build's status copy)."""
        chk = self._symmetry_check
        if chk is not None:
            c = chk.counters()
            self._symmetric = c["duplicate"] == 0 and c["out_of_box"] == 0
            self._symmetry_check = None
            # repeated coordinates need their rows folded before the map is transposed (two rows of
            # one coordinate reach the same (input, offset)); rows outside the box are not in the
            # brick index, so its duplicate count cannot see repeats among them: look at every row
            if (c["duplicate"] or c["out_of_box"]) and self._out_coords is not None:
                self.set_row_representatives(row_representatives(self._out_coords))
            self._out_coords = None
        return self._symmetric

    def set_row_representatives(self, rep: Optional[torch.Tensor]) -> "KernelMap":
        """Declare repeated output coordinates (``rep`` from ``row_representatives``, or None)."""
        assert self.invnbr is None, "set the representatives before the transposed map is built"
        self.row_rep = rep
        if rep is not None:
            self._symmetric = False
        return self
    @property
    def mask_words(self) -> int:
        return _mask_words(self.K)

    @property
    def neighbor_indices(self) -> torch.Tensor:
        """(N_out, K) view, the reference's layout (``conv.py:12-75``)."""
        return torch.as_strided(self.nbr, (self.n_out, self.K), (self.r_stride, self.k_stride))

    def ensure_inverse(self) -> "KernelMap":
        if self.invnbr is not None:
            return self
        dev = self.nbr.device
        W = self.mask_words
        need_out = self.out_masks is None
        if need_out:
            self.out_masks = torch.empty((self.n_out, W), dtype=torch.int32, device=dev)
        src, ks, rs = self.nbr, self.k_stride, self.r_stride
        if self.row_rep is not None:
            if need_out:  # the forward's masks come from the whole map
                self._invert(src, ks, rs, self.out_masks, None)
                need_out = False
            keep = self.row_rep == torch.arange(self.n_out, dtype=self.row_rep.dtype, device=dev)
            full = torch.as_strided(self.nbr, (self.K, self.n_out), (self.k_stride, self.r_stride))
            src, ks, rs = torch.where(keep[None, :], full, torch.full_like(full, -1)).contiguous(), self.n_out, 1
        self._conflicts = torch.zeros((1,), dtype=torch.int32, device=dev) if self.raw else None
        self.invnbr, self.in_masks = self._invert(src, ks, rs, self.out_masks if need_out else None,
                                                  self._conflicts)
        return self

    def _check_transposable(self) -> None:
        """Before the transposed map feeds an input gradient: a caller's map must send each
        (input, offset) to at most one output (synchronises once, caller's maps only)."""
        c = self._conflicts
        if c is not None:
            self._conflicts = None
            n = int(c.item())
            if n:
                raise ValueError(
                    f"neighbor_indices sends one input row to several output rows through one offset ({n} "
                    "entries); the gather input gradient needs a convolution map, where each (input, offset) "
                    "feeds at most one output")

    def _invert(self, src, ks, rs, out_masks, conflicts):
        dev = src.device
        invnbr = _lib.fill_(torch.empty((self.K, self.n_in), dtype=torch.int32, device=dev), -1)
        in_masks = _lib.fill_(torch.empty((self.n_in, self.mask_words), dtype=torch.int32, device=dev), 0)
        _lib.call("st_kmap_invert", _lib.ptr(src), ks, rs, self.n_out, self.K, self.n_in, _lib.ptr(invnbr),
                  _lib.ptr(in_masks), _lib.ptr(out_masks), _lib.ptr(conflicts), _lib.stream_of(dev))
        return invnbr, in_masks

    def fold_output_rows(self, dY: torch.Tensor) -> torch.Tensor:
        """dY summed over the rows of each repeated output coordinate into its lowest row (the
        row the transposed map holds); dY itself when no coordinate repeats."""
        if self.row_rep is None:
            return dY
        acc = torch.zeros(dY.shape, dtype=torch.float32, device=dY.device)
        acc.index_add_(0, self.row_rep.long(), dY.float())
        return acc.to(dY.dtype)

    def ensure_out_masks(self) -> "KernelMap":
        if self.out_masks is None:
            self.ensure_inverse()
        return self

    # ------------------------------------------------------------ GEMM plans
    def _build_plans(self, chunk: int) -> None:
        """Row order + tile plan of the forward (and with chunk != 0 the pair list and its chunk
        order, on the library's side stream, joined back before the call's work ends): one
        ``st_kmap_plans`` call over one buffer."""
        self.ensure_out_masks()
        plan = MapPlan.build(self.nbr, self.k_stride, self.r_stride, self.out_masks, self.K, self.n_out, self.n_in,
                             chunk)
        self._fwd_tiles = plan.tiles
        if chunk != 0:
            self._pairs[chunk] = plan.pairs

    def forward_plan(self) -> "TileMap":
        """Mask-sorted order of the output rows (forward): ``.perm`` of the forward tile plan."""
        return self.forward_tiles()

    def forward_tiles(self, with_pairs: bool = False) -> "TileMap":
        """Tile plan of the forward gather-GEMM (offsets and source rows per 128-row tile); with
        ``with_pairs`` the weight gradient's pair list is built in the same call."""
        if self._fwd_tiles is None:
            self._build_plans(_PAIR_CHUNK if with_pairs and _PAIR_CHUNK not in self._pairs else 0)
        return self._fwd_tiles

    def backward_tiles(self) -> "TileMap":
        """Tile plan of the input-gradient gather-GEMM (the forward's for a symmetric map)."""
        if self.symmetric:
            return self.forward_tiles()
        if self._bwd_tiles is None:
            self.ensure_inverse()
            self._check_transposable()
            self._bwd_tiles = MapPlan.build(self.invnbr, self.n_in, 1, self.in_masks, self.K, self.n_in, self.n_out,
                                            0).tiles
        return self._bwd_tiles

    def backward_plan(self) -> "TileMap":
        """Mask-sorted order of the input rows over the transposed map (input gradient)."""
        return self.backward_tiles()

    def pair_list(self, chunk: Optional[int] = None, with_tiles: bool = True) -> "PairList":
        """(in, out) pairs sorted by (offset, out) with equal-size chunks, for the weight gradient;
        the default chunk size comes with the forward tile plan unless ``with_tiles`` is False."""
        if chunk is None:
            chunk = _PAIR_CHUNK
        pl = self._pairs.get(chunk)
        if pl is None:
            if chunk == _PAIR_CHUNK and self._fwd_tiles is None and with_tiles:
                self._build_plans(chunk)
                return self._pairs[chunk]
            pl = PairList.build(self.nbr, self.k_stride, self.r_stride, self.n_out, self.K, self.n_in, chunk)
            self._pairs[chunk] = pl
        return pl

    def prepare(self) -> "KernelMap":
        """Build everything forward and backward need (idempotent): the tile plans and the pair
        list, the latter alongside the former on a side stream."""
        self.forward_tiles(with_pairs=True)
        self.backward_tiles()
        self.pair_list()
        return self

    def num_pairs(self) -> int:
        """Number of valid (input, output, offset) triples (synchronises)."""
        return int((self.neighbor_indices >= 0).sum().item())

    def window_order(self, slab: int):
        """(rows, map): the output rows sorted by offset mask (its first word) within consecutive
        slabs of ``slab`` rows (int32, n_out) and the map's columns in that order ((K, n_out)
        int32), kept per slab size -- the column order of the window weight gradient.  It skips
        an offset's 32-column steps without pairs, and in this order most steps of an offset
        have pairs in all columns or in none, while the rows of a slab stay near each other
        (config 5: 1.04x the useful MFMA rows at 4,096-row slabs, 1.29x in row order)."""
        got = self._window_orders.get(slab)
        if got is None:
            self.ensure_out_masks()
            m = self.out_masks[:, 0].to(torch.int64) & 0xFFFFFFFF
            pos = torch.arange(self.n_out, device=m.device, dtype=torch.int64)
            order = torch.sort((pos // slab) * (1 << 32) + m, stable=True).indices
            full = torch.as_strided(self.nbr, (self.K, self.n_out), (self.k_stride, self.r_stride))
            got = (order.to(torch.int32), full.index_select(1, order).contiguous())
            self._window_orders[slab] = got
        return got

    def triples(self) -> torch.Tensor:
        """(P, 3) int64 rows (in, out, k) sorted -- the canonical parity form."""
        nb = self.neighbor_indices.long()
        o, k = torch.nonzero(nb >= 0, as_tuple=True)
        t = torch.stack([nb[o, k], o, k], dim=1)
        key = (t[:, 0] * (self.n_out + 1) + t[:, 1]) * (self.K + 1) + t[:, 2]
        return t[torch.argsort(key)]


def row_representatives(coords: torch.Tensor) -> Optional[torch.Tensor]:
    """For (N, 4) coordinates with repeats: int32 (N,) lowest row holding each row's coordinate;
    None when every coordinate is unique (synchronises: only the repeated-coordinate path
    calls it)."""
    n = coords.shape[0]
    c = coords.to(torch.int64)
    key = (c[:, 0] << 48) | ((c[:, 1] & 0xFFFF) << 32) | ((c[:, 2] & 0xFFFF) << 16) | (c[:, 3] & 0xFFFF)
    uniq, inv = torch.unique(key, return_inverse=True)
    if uniq.shape[0] == n:
        return None
    rows = torch.arange(n, dtype=torch.int64, device=coords.device)
    first = torch.full((uniq.shape[0],), n, dtype=torch.int64, device=coords.device)
    first.scatter_reduce_(0, inv, rows, reduce="amin")
    return first[inv].to(torch.int32)


# pairs per weight-gradient task: ST_PAIR_CHUNK_AUTO, chosen on the GPU from the pair count P
# (the least power of two >= 1024 with at most 2048 chunks' worth of pairs): small lists keep
# 1024-pair tasks for parallelism, large ones take longer tasks and fewer partial sums
_PAIR_CHUNK = -1

# st_kmap_plans_layout fields (include/sparsetriton_amd.h)
(_PL_PERM, _PL_TILE_NK, _PL_TILE_KLIST, _PL_TILE_MAP, _PL_PAIRS, _PL_KSTART, _PL_CSTART, _PL_CORDER, _PL_BYTES,
 _PL_SCRATCH_BYTES, _PL_TILES, _PL_MAX_CHUNKS) = range(12)


@functools.lru_cache(maxsize=256)
def _plan_layout(n: int, K: int, chunk: int) -> tuple:
    arr = (ctypes.c_int64 * 12)()
    _lib.call("st_kmap_plans_layout", n, K, chunk, arr)
    return tuple(arr)


def _buf_view(buf: torch.Tensor, off: int, count: int, dtype: torch.dtype) -> torch.Tensor:
    size = torch.tensor([], dtype=dtype).element_size()
    return buf[off:off + count * size].view(dtype)


class TileMap:
    """Per-tile offsets and source rows of a gather-GEMM, in the tile order of the row order
    ``perm`` (n): ``nk`` (ntiles), ``klist`` (ntiles, K) int16, ``tmap`` (ntiles, K, 128) int32.
    ``*_ptr`` are the device addresses the GEMM entry points take; the tensors are views made
    on first use."""

    def __init__(self, perm, nk, klist, tmap):
        self._perm, self._nk, self._klist, self._tmap = perm, nk, klist, tmap
        self.perm_ptr, self.nk_ptr, self.klist_ptr, self.tmap_ptr = (t.data_ptr() for t in (perm, nk, klist, tmap))

    @classmethod
    def in_plan(cls, buf: torch.Tensor, L: tuple, n: int, K: int) -> "TileMap":
        tm = cls.__new__(cls)
        tm._buf, tm._L, tm._n, tm._K = buf, L, n, K
        tm._perm = tm._nk = tm._klist = tm._tmap = None
        base = buf.data_ptr()
        tm.perm_ptr, tm.nk_ptr = base + L[_PL_PERM], base + L[_PL_TILE_NK]
        tm.klist_ptr, tm.tmap_ptr = base + L[_PL_TILE_KLIST], base + L[_PL_TILE_MAP]
        return tm

    @property
    def perm(self) -> torch.Tensor:
        if self._perm is None:
            self._perm = _buf_view(self._buf, self._L[_PL_PERM], self._n, torch.int32)
        return self._perm

    @property
    def nk(self) -> torch.Tensor:
        if self._nk is None:
            self._nk = _buf_view(self._buf, self._L[_PL_TILE_NK], self._L[_PL_TILES], torch.int32)
        return self._nk

    @property
    def klist(self) -> torch.Tensor:
        if self._klist is None:
            self._klist = _buf_view(self._buf, self._L[_PL_TILE_KLIST], self._L[_PL_TILES] * self._K, torch.int16)
        return self._klist

    @property
    def tmap(self) -> torch.Tensor:
        if self._tmap is None:
            self._tmap = _buf_view(self._buf, self._L[_PL_TILE_MAP], self._L[_PL_TILES] * self._K * _lib.TILE_ROWS,
                                   torch.int32)
        return self._tmap

    @classmethod
    def build(cls, map_t, k_stride, r_stride, masks, K, perm, n_dst, n_src) -> "TileMap":
        """Tile plan of a given row order (``st_tile_plan``)."""
        dev = map_t.device
        nt = max((n_dst + _lib.TILE_ROWS - 1) // _lib.TILE_ROWS, 1)
        # one allocation: nk (nt) | klist (nt * K int16) | tmap (nt * K * 128), tmap on a 256-byte boundary
        kw = (nt * K + 1) // 2
        hdr = (nt + kw + 63) // 64 * 64
        buf = torch.empty((hdr + nt * K * _lib.TILE_ROWS,), dtype=torch.int32, device=dev)
        nk = buf[:nt]
        klist = buf[nt:nt + kw].view(torch.int16)[:nt * K]
        tmap = buf[hdr:]
        _lib.call("st_tile_plan", _lib.ptr(map_t), k_stride, r_stride, _lib.ptr(masks), _mask_words(K), K,
                  _lib.ptr(perm), n_dst, n_src, _lib.ptr(nk), _lib.ptr(klist), _lib.ptr(tmap), _lib.stream_of(dev))
        return cls(perm, nk, klist, tmap)


class PairList:
    """(in, out) int32 pairs sorted by (offset, out); ``kstart`` / ``cstart`` (K + 1) the first pair /
    chunk of each offset; ``max_chunks`` bounds the chunk count without reading it back;
    ``corder`` the chunk ids sorted by their first output row (the weight gradient's order).
    ``chunk`` is the size given to the builder; for -1 (chosen on the GPU) the size sits in the
    device word after ``cstart`` (``chunk_size()`` reads it back)."""

    def __init__(self, pairs, kstart, cstart, chunk, max_chunks, corder):
        self._pairs, self._kstart, self._cstart, self._corder = pairs, kstart, cstart, corder
        self.chunk, self.max_chunks = int(chunk), int(max_chunks)
        self.pairs_ptr, self.kstart_ptr, self.cstart_ptr, self.corder_ptr = (
            t.data_ptr() for t in (pairs, kstart, cstart, corder))

    @classmethod
    def in_plan(cls, buf: torch.Tensor, L: tuple, n: int, K: int, chunk: int) -> "PairList":
        pl = cls.__new__(cls)
        pl._buf, pl._L, pl._n, pl._K = buf, L, n, K
        pl._pairs = pl._kstart = pl._cstart = pl._corder = None
        pl.chunk, pl.max_chunks = int(chunk), int(L[_PL_MAX_CHUNKS])
        base = buf.data_ptr()
        pl.pairs_ptr, pl.kstart_ptr = base + L[_PL_PAIRS], base + L[_PL_KSTART]
        pl.cstart_ptr, pl.corder_ptr = base + L[_PL_CSTART], base + L[_PL_CORDER]
        return pl

    @property
    def pairs(self) -> torch.Tensor:
        if self._pairs is None:
            self._pairs = _buf_view(self._buf, self._L[_PL_PAIRS], 2 * max(self._K * self._n, 1), torch.int32)
        return self._pairs

    @property
    def kstart(self) -> torch.Tensor:
        if self._kstart is None:
            self._kstart = _buf_view(self._buf, self._L[_PL_KSTART], self._K + 1, torch.int32)
        return self._kstart

    @property
    def cstart(self) -> torch.Tensor:
        if self._cstart is None:
            self._cstart = _buf_view(self._buf, self._L[_PL_CSTART], self._K + 1, torch.int32)
        return self._cstart

    @property
    def corder(self) -> torch.Tensor:
        if self._corder is None:
            self._corder = _buf_view(self._buf, self._L[_PL_CORDER], self.max_chunks, torch.int32)
        return self._corder

    @classmethod
    def build(cls, map_t, k_stride, r_stride, n_out, K, n_in, chunk) -> "PairList":
        """A pair list with its own chunk size (``st_kmap_pairs`` + its chunk order)."""
        dev = map_t.device
        nb = ctypes.c_int64()
        _lib.call("st_kmap_pairs_sizes", n_out, K, ctypes.byref(nb))
        cap = K * n_out
        counts = torch.empty((K * nb.value + 1,), dtype=torch.int32, device=dev)
        kstart = torch.empty((K + 1,), dtype=torch.int32, device=dev)
        cstart = torch.empty((K + 2,), dtype=torch.int32, device=dev)
        pairs = torch.empty((2 * max(cap, 1),), dtype=torch.int32, device=dev)
        _lib.call("st_kmap_pairs", _lib.ptr(map_t), k_stride, r_stride, n_out, K, n_in, _lib.ptr(counts), nb.value,
                  int(chunk), _lib.ptr(kstart), _lib.ptr(cstart), _lib.ptr(pairs), cap, _lib.stream_of(dev))
        max_chunks = _plan_layout(int(n_out), int(K), int(chunk))[_PL_MAX_CHUNKS]
        corder = torch.empty((max(max_chunks, 1),), dtype=torch.int32, device=dev)
        if max_chunks <= _CHUNK_ORDER_MAX and K <= _CHUNK_ORDER_MAX_K:
            _lib.call("st_kmap_pairs_chunk_order", _lib.ptr(pairs), _lib.ptr(kstart), _lib.ptr(cstart), K, int(chunk),
                      max_chunks, n_out, _lib.ptr(corder), _lib.stream_of(dev))
        else:
            keys = torch.empty((max_chunks, 1), dtype=torch.int32, device=dev)
            _lib.call("st_kmap_pairs_chunk_keys", _lib.ptr(pairs), _lib.ptr(kstart), _lib.ptr(cstart), K, int(chunk),
                      max_chunks, n_out, _lib.ptr(keys), _lib.stream_of(dev))
            corder = TilePlan.build(max_chunks, 9, keys).perm
        pl = cls(pairs, kstart, cstart[:K + 1], int(chunk), max_chunks, corder)
        pl._size_word = cstart[K + 1:]
        return pl

    def chunk_size(self) -> int:
        """Pairs per chunk (reads the device word back for a list that chose its own size)."""
        if self.chunk > 0:
            return self.chunk
        word = getattr(self, "_size_word", None)
        if word is None:
            word = _buf_view(self._buf, self._L[_PL_CSTART] + 4 * (self._K + 1), 1, torch.int32)
        return int(word.item())


_CHUNK_ORDER_MAX, _CHUNK_ORDER_MAX_K = 16384, 28  # st_kmap_pairs_chunk_order's limits


class MapPlan:
    """The buffers of one ``st_kmap_plans`` call: ``tiles`` (TileMap) and, when built with a
    chunk size, ``pairs`` (PairList), all views of one allocation."""

    def __init__(self, tiles: TileMap, pairs: Optional[PairList]):
        self.tiles, self.pairs = tiles, pairs

    @classmethod
    def build(cls, map_t, k_stride, r_stride, masks, K, n_dst, n_src, chunk) -> "MapPlan":
        dev = map_t.device
        L = _plan_layout(int(n_dst), int(K), int(chunk))
        buf = torch.empty((L[_PL_BYTES],), dtype=torch.uint8, device=dev)
        scratch = torch.empty((L[_PL_SCRATCH_BYTES],), dtype=torch.uint8, device=dev)
        _lib.call("st_kmap_plans", map_t.data_ptr(), k_stride, r_stride, masks.data_ptr(), K, n_dst, n_src, chunk,
                  get_tile_slab_bits(), buf.data_ptr(), scratch.data_ptr(), _lib.stream_of(dev))
        return cls(TileMap.in_plan(buf, L, n_dst, K),
                   PairList.in_plan(buf, L, n_dst, K, chunk) if chunk != 0 else None)


@functools.lru_cache(maxsize=64)
def _sort_workspace_bytes(n: int) -> int:
    nbytes = ctypes.c_size_t()
    _lib.call("st_kmap_sort_workspace", n, ctypes.byref(nbytes))
    return max(int(nbytes.value), 1)


class TilePlan:
    """Destination-row order of a gather-GEMM: ``perm`` (n) lists the rows sorted by their
    offset bitmask, so 16/32-row MFMA slabs hold rows that need the same offsets."""

    def __init__(self, perm: torch.Tensor):
        self.perm = perm

    @classmethod
    def build(cls, n, K, masks) -> "TilePlan":
        dev = masks.device
        W = _mask_words(K)
        nbytes = _sort_workspace_bytes(n)
        # one scratch allocation: keys (2n) | rows (n) | sort workspace; perm is kept
        scratch = torch.empty((3 * n + (nbytes + 3) // 4,), dtype=torch.int32, device=dev)
        perm = torch.empty((n,), dtype=torch.int32, device=dev)
        _lib.call("st_kmap_sort_rows", _lib.ptr(masks), W, K, n, scratch.data_ptr(), scratch.data_ptr() + 8 * n,
                  _lib.ptr(perm), scratch.data_ptr() + 12 * n, nbytes, _lib.stream_of(dev))
        return cls(perm)


# ----------------------------------------------------------------- builders

def _offsets_i32(kernel_offsets: torch.Tensor) -> torch.Tensor:
    return kernel_offsets.to(torch.int32).contiguous()


def query_kernel_map(table: HashTable, out_coords: torch.Tensor, kernel_offsets: torch.Tensor, spatial_shape,
                     stride: int, n_in: int, symmetric: bool = False) -> KernelMap:
    """nbr[k, o] = row of out_o * stride - t_k (bounds [0, shape)), via ``st_kmap_query`` (hash table).

    ``symmetric`` declares a submanifold map of an odd kernel (offsets ``t`` and
    ``-t`` at k and K-1-k) over the table's own coordinates, whose transpose is
    the map itself read backwards when those coordinates are unique and inside
    ``spatial_shape``: the query counts rows outside it into the table's status
    words (the table build counts repeats), and the map checks both counts
    before it first relies on the claim."""
    out_coords = out_coords.contiguous()
    dev = out_coords.device
    _lib.require_device(out_coords, "out_coords")
    n_out = out_coords.shape[0]
    K = kernel_offsets.shape[0]
    if K > _lib.MAX_KVOL:
        raise ValueError(f"kernel volume {K} exceeds the supported maximum {_lib.MAX_KVOL}")
    nbr = torch.empty((K, n_out), dtype=torch.int32, device=dev)
    masks = torch.empty((n_out, _mask_words(K)), dtype=torch.int32, device=dev)
    sx, sy, sz = (int(v) for v in spatial_shape)
    status = table.status_tensor() if symmetric else None
    keys, vals = table.table_keys, table.table_values  # runs a deferred insert first
    offs = _offsets_i32(kernel_offsets)  # held until the launch is queued (it may be a temporary)
    _lib.call("st_kmap_query", _lib.ptr(out_coords), _lib.coord_code(out_coords.dtype), n_out, _lib.ptr(offs), K,
              int(stride), sx, sy, sz, _lib.ptr(keys), _lib.ptr(vals), table.capacity, _lib.ptr(nbr), n_out, 1,
              _lib.ptr(masks), _lib.ptr(status), _lib.stream_of(dev))
    check = table.snapshot() if symmetric else None
    km = KernelMap(nbr, n_in, n_out, K, out_masks=masks, symmetric=symmetric, symmetry_check=check)
    km._out_coords = out_coords if symmetric else None
    return km


@functools.lru_cache(maxsize=64)
def _subm_workspace_bytes(n: int, batches: int, sx: int, sy: int, sz: int) -> int:
    nbytes = ctypes.c_int64()
    rc = _lib.lib().st_kmap_subm_workspace(n, batches, sx, sy, sz, ctypes.byref(nbytes))
    return int(nbytes.value) if rc == _lib.ST_OK else -1


def subm_kernel_map(coords: torch.Tensor, batch_size: int, spatial_shape, kernel_offsets: torch.Tensor,
                    symmetric: bool = True):
    """Submanifold map of ``coords`` over themselves (out = in, stride 1, bounds ``spatial_shape``) by
    ``st_kmap_subm``, which indexes the coordinates by 4x4x4 bricks (no hash table).

    Returns (KernelMap, StatusSnapshot of the build's bad-coordinate / duplicate / out-of-box counts), or
    None when the box cannot be indexed (batch or shape out of range, or far larger than the set) -- the
    caller then queries a hash table."""
    from sparsetriton_amd.utils.hash import StatusSnapshot

    coords = coords.contiguous()
    dev = coords.device
    _lib.require_device(coords, "coordinates")
    n = coords.shape[0]
    K = kernel_offsets.shape[0]
    if K > _lib.MAX_KVOL:
        raise ValueError(f"kernel volume {K} exceeds the supported maximum {_lib.MAX_KVOL}")
    sx, sy, sz = (int(v) for v in spatial_shape)
    nbytes = _subm_workspace_bytes(int(n), int(batch_size), sx, sy, sz)
    if nbytes < 0:
        return None
    work = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    # cleared by the launch (which an empty set skips)
    status = (torch.empty if n else torch.zeros)((_lib.STATUS_WORDS,), dtype=torch.int32, device=dev)
    nbr = torch.empty((K, n), dtype=torch.int32, device=dev)
    masks = torch.empty((n, _mask_words(K)), dtype=torch.int32, device=dev)
    offs = _offsets_i32(kernel_offsets)  # held until the launch is queued (it may be a temporary)
    rc = _lib.lib().st_kmap_subm(_lib.ptr(coords), _lib.coord_code(coords.dtype), n, _lib.ptr(offs), K,
                                 int(batch_size), sx, sy, sz,
                                 _lib.ptr(work), nbytes, _lib.ptr(nbr), _lib.ptr(masks), _lib.ptr(status),
                                 _lib.stream_of(dev))
    _lib.check(rc, "st_kmap_subm")
    snap = StatusSnapshot(status)
    km = KernelMap(nbr, n, n, K, out_masks=masks, symmetric=symmetric, symmetry_check=snap if symmetric else None)
    km._out_coords = coords if symmetric else None
    return km, snap



class BrickIndex:
    """Brick index of a coordinate set over the box [0, batch_size) x [0, spatial_shape)
    (``st_subm_index``): what a submanifold lookup needs -- ``st_kmap_subm_query`` builds maps
    from it, ``st_subm_fly_gemm`` looks neighbours up in it inside the GEMM.  ``status`` (a
    StatusSnapshot) holds the build's bad-coordinate / duplicate / out-of-box counts."""

    def __init__(self, coords, batch_size, spatial_shape, work, nbytes, status):
        self.coords = coords
        self.geometry = (int(batch_size),) + tuple(int(v) for v in spatial_shape)
        self.work, self.nbytes, self.status = work, int(nbytes), status
        self._orders = {}

    @classmethod
    def build(cls, coords: torch.Tensor, batch_size: int, spatial_shape) -> Optional["BrickIndex"]:
        """The index, or None when the box cannot be indexed (see ``subm_kernel_map``)."""
        from sparsetriton_amd.utils.hash import StatusSnapshot

        coords = coords.contiguous()
        dev = coords.device
        _lib.require_device(coords, "coordinates")
        n = coords.shape[0]
        sx, sy, sz = (int(v) for v in spatial_shape)
        nbytes = _subm_workspace_bytes(int(n), int(batch_size), sx, sy, sz)
        if nbytes < 0:
            return None
        work = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=dev)
        status = (torch.empty if n else torch.zeros)((_lib.STATUS_WORDS,), dtype=torch.int32, device=dev)
        _lib.call("st_subm_index", _lib.ptr(coords), _lib.coord_code(coords.dtype), n, int(batch_size), sx, sy, sz,
                  _lib.ptr(work), nbytes, _lib.ptr(status), _lib.stream_of(dev))
        return cls(coords, batch_size, spatial_shape, work, nbytes, StatusSnapshot(status))

    @property
    def n(self) -> int:
        return self.coords.shape[0]

    def transposable(self) -> bool:
        """Whether a submanifold map of an odd kernel over these coordinates is its own transpose
        (offsets reversed): every coordinate unique and inside the box (waits for the counts)."""
        c = self.status.counters()
        return c["duplicate"] == 0 and c["out_of_box"] == 0

    def query(self, kernel_offsets: torch.Tensor) -> KernelMap:
        """The (K, n) submanifold map and its row masks from the index (``st_kmap_subm_query``)."""
        n = self.n
        K = kernel_offsets.shape[0]
        dev = self.coords.device
        nbr = torch.empty((K, n), dtype=torch.int32, device=dev)
        masks = torch.empty((n, _mask_words(K)), dtype=torch.int32, device=dev)
        offs = _offsets_i32(kernel_offsets)
        _lib.call("st_kmap_subm_query", _lib.ptr(self.coords), _lib.coord_code(self.coords.dtype), n, _lib.ptr(offs),
                  K, *self.geometry, _lib.ptr(self.work), self.nbytes, _lib.ptr(nbr), _lib.ptr(masks),
                  _lib.stream_of(dev))
        return KernelMap(nbr, n, n, K, out_masks=masks)

    def tile_order(self, kernel_offsets: torch.Tensor, key) -> torch.Tensor:
        """The rows sorted by their offset masks (``st_kmap_subm_query`` writing the masks only,
        then ``st_kmap_sort_rows``): the tile order ``st_subm_fly_gemm`` takes, so a 128-row tile
        holds rows that need the same offsets.  Built once per kernel geometry ``key`` and kept with
        the index (n int32; no map is stored)."""
        if key not in self._orders:
            n = self.n
            K = kernel_offsets.shape[0]
            dev = self.coords.device
            masks = torch.empty((n, _mask_words(K)), dtype=torch.int32, device=dev)
            offs = _offsets_i32(kernel_offsets)
            _lib.call("st_kmap_subm_query", _lib.ptr(self.coords), _lib.coord_code(self.coords.dtype), n,
                      _lib.ptr(offs), K, *self.geometry, _lib.ptr(self.work), self.nbytes, None, _lib.ptr(masks),
                      _lib.stream_of(dev))
            self._orders[key] = TilePlan.build(n, K, masks).perm
        return self._orders[key]


class OutCoordTable:
    """Dedup table of a strided / transposed build: output coordinate -> output row."""

    def __init__(self, keys: torch.Tensor, slot_out: torch.Tensor):
        self.table_keys = keys
        self.table_values = slot_out

    @property
    def capacity(self) -> int:
        return self.table_keys.shape[0]


def build_out_coords_and_map(in_coords: torch.Tensor, spatial_shape, kernel_size: int, stride: int, dilation: int,
                             padding: int, transposed: bool, in_table: Optional[HashTable] = None,
                             with_map: bool = True, chunk_size: Optional[int] = None):
    """Strided / transposed output coordinates plus (optionally) their kernel map.

    Returns (out_coords, new_spatial_shape, kernel_offsets, kmap_or_None, out_table).
    One host synchronisation reads the output count.

    ``chunk_size`` (offsets per chunk, the reference's ``kmap.py:270-278``)
    orders the candidates chunk by chunk, as the reference's loop does, and
    bounds the dedup table: it starts at twice the candidates of one chunk
    and doubles while it overflows (each retry one more pass over the
    inputs), so its size follows the distinct outputs rather than all
    candidates.  Without it the table is sized for every candidate up front,
    and still grows if that size was clamped to the 32-bit slot range.
    """
    dev = in_coords.device
    _lib.require_device(in_coords, "coordinates")
    in_coords = in_coords.contiguous()
    n = in_coords.shape[0]
    offsets = _target_offsets(kernel_size, dilation, padding, transposed, dev)
    kernel_offsets = offsets.to(in_coords.dtype, copy=True)  # returned to the caller: not the shared tensor
    K = offsets.shape[0]
    if K > _lib.MAX_KVOL:
        raise ValueError(f"kernel volume {K} exceeds the supported maximum {_lib.MAX_KVOL}")
    new_shape = out_spatial_shape(spatial_shape, kernel_size, stride, dilation, padding, transposed)
    g = _lib.OutGeom()
    g.K = K
    g.transposed = 1 if transposed else 0
    g.stride = int(stride)
    g.chunk = int(chunk_size) if chunk_size else 0
    for a in range(3):
        g.in_shape[a] = int(spatial_shape[a])
        g.out_shape[a] = int(new_shape[a])
    dcap, nblocks = ctypes.c_int64(), ctypes.c_int64()
    _lib.call("st_outcoords_sizes", n, ctypes.byref(g), int(kernel_size), int(dilation), ctypes.byref(dcap),
              ctypes.byref(nblocks))
    max_cap, nblocks = dcap.value, nblocks.value
    dcap = max_cap
    if chunk_size and 0 < int(chunk_size) < K:
        dcap = min(max_cap, 2 * n * int(chunk_size) + 64)
    s = _lib.stream_of(dev)
    counts = torch.empty((nblocks + 1,), dtype=torch.int32, device=dev)
    status = torch.empty((_lib.STATUS_WORDS,), dtype=torch.int32, device=dev)
    offs = _offsets_i32(offsets)
    while True:
        dkeys = _lib.fill_(torch.empty((dcap,), dtype=torch.int64, device=dev), -1)
        dvals = _lib.fill_(torch.empty((dcap,), dtype=torch.int32, device=dev), -1)
        _lib.fill_(status, 0)
        _lib.call("st_outcoords_plan", _lib.ptr(in_coords), _lib.coord_code(in_coords.dtype), n, _lib.ptr(offs),
                  ctypes.byref(g), _lib.ptr(dkeys), _lib.ptr(dvals), dcap, _lib.ptr(counts), nblocks,
                  _lib.ptr(status), s)
        tail = torch.stack([counts[nblocks], status[_lib.STATUS_OVERFLOW], status[_lib.STATUS_BAD_COORD]]).tolist()
        n_out, overflow, bad = tail
        if not overflow:
            break
        if dcap >= max_cap:
            raise RuntimeError(f"output-coordinate dedup table overflowed ({overflow} candidates dropped)")
        dcap = min(max_cap, 2 * dcap)
    if bad:
        raise RuntimeError(f"{bad} output coordinates fall outside the packable range")
    out_coords = torch.empty((n_out, 4), dtype=in_coords.dtype, device=dev)
    slot_out = torch.empty((dcap,), dtype=torch.int32, device=dev)
    kmap = None
    nbr = invnbr = out_masks = in_masks = None
    if with_map:
        W = _mask_words(K)
        nbr = _lib.fill_(torch.empty((K, n_out), dtype=torch.int32, device=dev), -1)
        invnbr = _lib.fill_(torch.empty((K, n), dtype=torch.int32, device=dev), -1)
        out_masks = _lib.fill_(torch.empty((n_out, W), dtype=torch.int32, device=dev), 0)
        in_masks = _lib.fill_(torch.empty((n, W), dtype=torch.int32, device=dev), 0)
    ik = iv = None
    icap = 0
    if in_table is not None:
        ik, iv, icap = in_table.table_keys, in_table.table_values, in_table.capacity
    _lib.call("st_outcoords_emit", _lib.ptr(in_coords), _lib.coord_code(in_coords.dtype), n, _lib.ptr(offs),
              ctypes.byref(g), _lib.ptr(dkeys), _lib.ptr(dvals), _lib.ptr(slot_out), dcap, _lib.ptr(counts), nblocks,
              _lib.ptr(ik), _lib.ptr(iv), icap, _lib.ptr(out_coords), n_out, _lib.ptr(nbr), _lib.ptr(invnbr),
              _lib.ptr(out_masks), _lib.ptr(in_masks), s)
    if with_map:
        kmap = KernelMap(nbr, n, n_out, K, out_masks=out_masks, invnbr=invnbr, in_masks=in_masks)
    return out_coords, torch.Size(new_shape), kernel_offsets, kmap, OutCoordTable(dkeys, slot_out)


def brick_out_coords_and_map(in_coords: torch.Tensor, batch_size: int, spatial_shape, kernel_size: int,
                             stride: int, dilation: int, padding: int, transposed: bool, with_map: bool = True,
                             chunk_size: Optional[int] = None):
    """``build_out_coords_and_map`` without hash tables: the same output coordinates in the same
    order and the same map, through brick indexes (``st_outcoords_brick_*`` over the candidates'
    output box, ``st_kmap_strided_query`` over the input coordinates' index).

    Returns (out_coords, new_spatial_shape, kernel_offsets, kmap_or_None, status) -- ``status``
    (a StatusSnapshot of the input index, or None without a map) carries the bad-coordinate count
    the input hash table would report -- or None when the boxes cannot be indexed or a row's
    batch index lies outside [0, batch_size); the caller then uses ``build_out_coords_and_map``.
    One host synchronisation reads the output count.
    """
    from sparsetriton_amd.utils.hash import StatusSnapshot

    dev = in_coords.device
    _lib.require_device(in_coords, "coordinates")
    in_coords = in_coords.contiguous()
    n = in_coords.shape[0]
    if n == 0 or batch_size < 1:
        return None
    offsets = _target_offsets(kernel_size, dilation, padding, transposed, dev)
    K = offsets.shape[0]
    if K > _lib.MAX_KVOL:
        raise ValueError(f"kernel volume {K} exceeds the supported maximum {_lib.MAX_KVOL}")
    new_shape = out_spatial_shape(spatial_shape, kernel_size, stride, dilation, padding, transposed)
    g = _lib.OutGeom()
    g.K = K
    g.transposed = 1 if transposed else 0
    g.stride = int(stride)
    g.chunk = int(chunk_size) if chunk_size else 0
    for a in range(3):
        g.in_shape[a] = int(spatial_shape[a])
        g.out_shape[a] = int(new_shape[a])
    in_bytes = _subm_workspace_bytes(int(n), int(batch_size), *(int(v) for v in spatial_shape)) if with_map else 0
    if in_bytes < 0:
        return None
    wbytes, nblocks = ctypes.c_int64(), ctypes.c_int64()
    rc = _lib.lib().st_outcoords_brick_sizes(n, ctypes.byref(g), int(batch_size), int(kernel_size), int(dilation),
                                            ctypes.byref(wbytes), ctypes.byref(nblocks))
    if rc == _lib.ERR_UNSUPPORTED:
        return None
    _lib.check(rc, "st_outcoords_brick_sizes")
    wbytes, nblocks = wbytes.value, nblocks.value
    s = _lib.stream_of(dev)
    cc = _lib.coord_code(in_coords.dtype)
    work = torch.empty((wbytes,), dtype=torch.uint8, device=dev)
    counts = torch.empty((nblocks + 1,), dtype=torch.int32, device=dev)
    status = torch.empty((_lib.STATUS_WORDS,), dtype=torch.int32, device=dev)
    offs = _offsets_i32(offsets)
    _lib.call("st_outcoords_brick_plan", _lib.ptr(in_coords), cc, n, _lib.ptr(offs), ctypes.byref(g),
              int(batch_size), int(kernel_size), int(dilation), _lib.ptr(work), wbytes, _lib.ptr(counts), nblocks,
              _lib.ptr(status), s)
    index = None
    if with_map:
        # the input index is queued before the host waits for the output count
        index = BrickIndex.build(in_coords, batch_size, spatial_shape)
    n_out, outside, over = torch.stack([counts[nblocks], status[_lib.STATUS_OUT_OF_BOX],
                                        status[_lib.STATUS_OVERFLOW]]).tolist()
    if outside or over:
        return None
    kernel_offsets = offsets.to(in_coords.dtype, copy=True)  # returned to the caller: not the shared tensor
    out_coords = torch.empty((n_out, 4), dtype=in_coords.dtype, device=dev)
    _lib.call("st_outcoords_brick_emit", _lib.ptr(in_coords), cc, n, _lib.ptr(offs), ctypes.byref(g),
              int(batch_size), int(kernel_size), int(dilation), _lib.ptr(work), wbytes, _lib.ptr(counts), nblocks,
              _lib.ptr(out_coords), n_out, s)
    if not with_map:
        return out_coords, torch.Size(new_shape), kernel_offsets, None, None
    W = _mask_words(K)
    nbr = torch.empty((K, n_out), dtype=torch.int32, device=dev)
    invnbr = torch.empty((K, n), dtype=torch.int32, device=dev)
    out_masks = torch.empty((n_out, W), dtype=torch.int32, device=dev)
    in_masks = torch.empty((n, W), dtype=torch.int32, device=dev)
    _lib.call("st_kmap_strided_query", _lib.ptr(out_coords), cc, n_out, _lib.ptr(offs), ctypes.byref(g),
              int(batch_size), _lib.ptr(index.work), index.nbytes, n, _lib.ptr(nbr), _lib.ptr(out_masks), s)
    _lib.call("st_outcoords_brick_inverse", _lib.ptr(in_coords), cc, n, _lib.ptr(offs), ctypes.byref(g),
              int(batch_size), int(kernel_size), int(dilation), _lib.ptr(work), wbytes, _lib.ptr(index.work),
              index.nbytes, _lib.ptr(invnbr), _lib.ptr(in_masks), s)
    kmap = KernelMap(nbr, n, n_out, K, out_masks=out_masks, invnbr=invnbr, in_masks=in_masks)
    return out_coords, torch.Size(new_shape), kernel_offsets, kmap, index.status


def build_out_coords(
    in_coords: torch.Tensor,
    spatial_shape,
    kernel_size: int,
    stride: int = 1,
    dilation: int = 1,
    padding: int = 1,
    transposed: bool = False,
    submanifold: bool = True,
    chunk_size: int = None,
):
    """(out_coords, new_spatial_shape, kernel_offsets) of a sparse convolution (``kmap.py:447-495``).

    Submanifold with stride 1 and centred padding returns the input
    coordinates unchanged (``kmap.py:261-262``).  Otherwise candidates
    ``in + t_k`` (or ``in * s + t_k`` transposed) pass the stride and range
    filters and are deduplicated, in first-occurrence order of the
    input-major / offset-minor candidate enumeration -- with ``chunk_size``
    offsets per chunk, chunk by chunk as the reference's loop
    (``kmap.py:270-278``).  Deduplication runs through a brick index of the
    candidates' output box (``brick_out_coords_and_map``), or, where the box
    cannot be indexed, a hash table sized by the distinct outputs (see
    ``build_out_coords_and_map``).  Candidates are never materialised.
    """
    offsets = _target_offsets(kernel_size, dilation, padding, transposed, in_coords.device).to(in_coords.dtype)
    if submanifold and stride == 1 and ((kernel_size - 1) * dilation) // 2 == padding:
        return in_coords, spatial_shape, offsets
    if in_coords.shape[0] > 0:
        # the brick build needs the batch count: one read of the largest batch index
        batches = int(in_coords[:, 0].max().item()) + 1
        built = brick_out_coords_and_map(in_coords, batches, spatial_shape, kernel_size, stride, dilation, padding,
                                         transposed, with_map=False, chunk_size=chunk_size)
        if built is not None:
            return built[0], built[1], built[2]
    out_coords, new_shape, kernel_offsets, _, _ = build_out_coords_and_map(
        in_coords, spatial_shape, kernel_size, stride, dilation, padding, transposed, with_map=False,
        chunk_size=chunk_size)
    return out_coords, new_shape, kernel_offsets
