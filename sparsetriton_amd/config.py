"""Process-wide settings read by the sparse-convolution path at call time.

Mirrors the reference's setter/getter surface (``sparsetriton/config.py:21-201``)
so user code that flips the algorithm or the coordinate dtype keeps working:

* ``ConvAlgo`` -- same two members and string values (``config.py:34-35``).
* coordinate dtype (default ``torch.int16``), hash-table size factor (1.5),
  maximum probe count (16) -- same defaults (``config.py:38-43``) and the same
  validation errors (``TypeError`` / ``AssertionError`` with the same messages).

Differences in meaning, both deliberate:

* The hash table built by this package sizes itself as
  ``max(factor, MIN_TABLE_FACTOR) * N`` slots.  Open addressing on exact 64-bit
  keys needs a load factor at or below one half to keep miss chains short;
  the reference's 1.5 gives 0.67.
* ``h_tbl_max_probe_n`` is kept for API compatibility only.  The reference
  never reads it either (its kernels hard-code 128 probes, ``utils/hash.py:211``);
  this package's probes are bounded by the table size, so an insert can only
  fail when the table is full, and that failure is reported, not dropped.

One addition: ``set_fp32_precision`` picks how fp32 convolutions use the
matrix cores.  The reference's fp32 ``tl.dot`` runs in TF32 on NVIDIA GPUs
(10-bit mantissa products).  Here the default ``"bf16x3"`` splits each fp32
operand into two bf16 parts and sums three bf16 MFMA products (relative error
per product about 2^-15, fp32 accumulation); ``"ieee"`` uses the fp32 MFMA
instructions (one-sixteenth of the bf16 rate on gfx950).
"""

from enum import Enum

import torch

__all__ = [
    "ConvAlgo",
    "set_coords_dtype",
    "get_coords_dtype",
    "set_conv_algo",
    "get_conv_algo",
    "set_h_table_f",
    "get_h_table_f",
    "set_h_table_max_p",
    "get_h_table_max_p",
    "set_fp32_precision",
    "get_fp32_precision",
    "FP32_PRECISIONS",
    "set_tile_slab_bits",
    "get_tile_slab_bits",
    "MIN_TABLE_FACTOR",
]

FP32_PRECISIONS = ("bf16x3", "ieee")

# Lowest slots-per-key ratio the hash table is built with (load factor 0.5).
MIN_TABLE_FACTOR = 2.0


class ConvAlgo(Enum):
    """Convolution algorithm switch, read by ``sparse_conv3d`` on every call.

    ``PrecomputedNeighborGEMM`` builds an offset-major kernel map once per
    coordinate set and runs gather-GEMM kernels over it.
    ``ImplicitHashFlyGEMM`` skips the map and probes the coordinate hash table
    inside the GEMM kernels.
    """

    ImplicitHashFlyGEMM = "Implicit_hashfly_gemm"
    PrecomputedNeighborGEMM = "Precomputed_neighbor_gemm"


_STATE: dict = {
    "coords_dtype": torch.int16,
    "algo": ConvAlgo.PrecomputedNeighborGEMM,
    "h_tbl_factor": 1.5,
    "h_tbl_max_probe_n": 16,
    "fp32_precision": "bf16x3",
    "tile_slab_bits": 0,
}


def set_coords_dtype(dtype: torch.dtype) -> None:
    """Set the integer dtype that ``SparseTensor`` casts coordinates to."""
    if not isinstance(dtype, torch.dtype):
        raise TypeError(f"Expected torch.dtype, got {type(dtype)}")
    _STATE["coords_dtype"] = dtype


def get_coords_dtype() -> torch.dtype:
    """Return the coordinate dtype (default ``torch.int16``)."""
    return _STATE["coords_dtype"]


def set_conv_algo(algo: ConvAlgo) -> None:
    """Select the convolution algorithm used by subsequent ``sparse_conv3d`` calls."""
    if not isinstance(algo, ConvAlgo):
        raise TypeError(f"Expected ConvAlgo, got {type(algo)}")
    _STATE["algo"] = algo


def get_conv_algo() -> ConvAlgo:
    """Return the selected convolution algorithm."""
    return _STATE["algo"]


def set_h_table_f(factor) -> None:
    """Set the hash-table slots-per-key factor (must be >= 1)."""
    try:
        value = float(factor)
    except (TypeError, ValueError):
        raise TypeError("factor must be a number")
    assert value >= 1, "factor must be >= 1"
    _STATE["h_tbl_factor"] = value


def get_h_table_f() -> float:
    """Return the hash-table slots-per-key factor."""
    return _STATE["h_tbl_factor"]


def set_h_table_max_p(probe_n) -> None:
    """Set the (compatibility-only) maximum probe count; must be positive."""
    try:
        value = int(probe_n)
    except (TypeError, ValueError):
        raise TypeError("probe_n must be an integer")
    assert value > 0, "probe_n must be positive"
    _STATE["h_tbl_max_probe_n"] = value


def get_h_table_max_p() -> int:
    """Return the (compatibility-only) maximum probe count."""
    return _STATE["h_tbl_max_probe_n"]


def set_fp32_precision(precision: str) -> None:
    """Matrix-core arithmetic of fp32 convolutions: ``"bf16x3"`` (default) or ``"ieee"``."""
    if precision not in FP32_PRECISIONS:
        raise ValueError(f"fp32 precision must be one of {FP32_PRECISIONS}, got {precision!r}")
    _STATE["fp32_precision"] = precision


def get_fp32_precision() -> str:
    """Current fp32 matrix-core arithmetic (``"bf16x3"`` or ``"ieee"``)."""
    return _STATE["fp32_precision"]


def set_tile_slab_bits(bits: int) -> None:
    """Group the gather-GEMM's destination rows into 2**bits slabs of their row order before
    sorting them by offset mask (0..8; 0 = one slab).  With rows in spatial order the tiles that
    run together then gather from one slab of input rows, which stays in L2, at the price of
    tiles that mix more masks.  Read when a kernel map's plans are built."""
    bits = int(bits)
    assert 0 <= bits <= 8, "tile slab bits must be in [0, 8]"
    _STATE["tile_slab_bits"] = bits


def get_tile_slab_bits() -> int:
    return _STATE["tile_slab_bits"]
