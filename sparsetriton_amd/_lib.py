"""ctypes binding of libsparsetriton_amd.so (declared in include/sparsetriton_amd.h).

The library is the only compute path for the sparse-convolution kernels:
there is no CPU or PyTorch fallback.  ``lib()`` raises ``RuntimeError`` when
the library is missing or cannot be loaded, and every wrapper raises when the
C call returns an error code.
"""

import ctypes
import os
from pathlib import Path

import torch

_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libsparsetriton_amd.so"

ST_OK = 0
ERR_UNSUPPORTED = -3
ERRORS = {-1: "invalid argument", -2: "HIP runtime error", -3: "unsupported dtype or size"}

COORD_DTYPES = {torch.int16: 0, torch.int32: 1, torch.int64: 2}
FEAT_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

STATUS_WORDS = 4
STATUS_OVERFLOW, STATUS_BAD_COORD, STATUS_DUPLICATE, STATUS_OUT_OF_BOX = 0, 1, 2, 3

W_TRANSPOSE, W_REVERSE, W_COPY = 0, 1, 2
GATHER_REVERSE_K = 1
COLUMN_SUM_NOALLOC_MAX_C = 2048
MAX_KVOL = 512
TILE_ROWS = 128


class OutGeom(ctypes.Structure):
    _fields_ = [
        ("K", ctypes.c_int32),
        ("transposed", ctypes.c_int32),
        ("stride", ctypes.c_int64),
        ("in_shape", ctypes.c_int64 * 3),
        ("out_shape", ctypes.c_int64 * 3),
        ("chunk", ctypes.c_int64),
    ]


class Lookup(ctypes.Structure):
    _fields_ = [
        ("K", ctypes.c_int32),
        ("sign", ctypes.c_int32),
        ("mul", ctypes.c_int64),
        ("div", ctypes.c_int64),
        ("bounds", ctypes.c_int64 * 3),
        ("row_bounds", ctypes.c_int64 * 3),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64

# name -> argtypes (all functions return int unless listed in _RESTYPES)
_SIGNATURES = {
    "st_version": [],
    "st_mfma_peak": [_I, _I, _P, ctypes.POINTER(ctypes.c_int64), _P],
    "st_fill_u32": [_P, _L, ctypes.c_uint32, _P],
    "st_fill_u64": [_P, _L, ctypes.c_uint64, _P],
    "st_hash_probe_mode": [_I],
    "st_hash_insert": [_P, _I, _L, _L, _P, _P, _L, _P, _P],
    "st_hash_build_workspace": [_L, _L, ctypes.POINTER(_L)],
    "st_hash_build": [_P, _I, _L, _L, _P, _P, _L, _I, _P, _L, _P, _P],
    "st_hash_query": [_P, _I, _L, _P, _P, _L, _P, _P],
    "st_kmap_query": [_P, _I, _L, _P, _I, _L, _L, _L, _L, _P, _P, _L, _P, _L, _L, _P, _P, _P],
    "st_kmap_subm_workspace": [_L, _L, _L, _L, _L, ctypes.POINTER(_L)],
    "st_kmap_subm": [_P, _I, _L, _P, _I, _L, _L, _L, _L, _P, _L, _P, _P, _P, _P],
    "st_subm_index": [_P, _I, _L, _L, _L, _L, _L, _P, _L, _P, _P],
    "st_kmap_subm_query": [_P, _I, _L, _P, _I, _L, _L, _L, _L, _P, _L, _P, _P, _P],
    "st_subm_fly_ok": [_L, _I, _I, _I, _I],
    "st_subm_fly_gemm": [_P, _P, _I, _L, _P, _I, _L, _L, _L, _L, _P, _L, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "st_outcoords_sizes": [_L, ctypes.POINTER(OutGeom), _L, _L, ctypes.POINTER(_L), ctypes.POINTER(_L)],
    "st_outcoords_plan": [_P, _I, _L, _P, ctypes.POINTER(OutGeom), _P, _P, _L, _P, _L, _P, _P],
    "st_outcoords_emit": [_P, _I, _L, _P, ctypes.POINTER(OutGeom), _P, _P, _P, _L, _P, _L, _P, _P, _L, _P, _L,
                          _P, _P, _P, _P, _P],
    "st_outcoords_brick_sizes": [_L, ctypes.POINTER(OutGeom), _L, _L, _L, ctypes.POINTER(_L), ctypes.POINTER(_L)],
    "st_outcoords_brick_plan": [_P, _I, _L, _P, ctypes.POINTER(OutGeom), _L, _L, _L, _P, _L, _P, _L, _P, _P],
    "st_outcoords_brick_emit": [_P, _I, _L, _P, ctypes.POINTER(OutGeom), _L, _L, _L, _P, _L, _P, _L, _P, _L, _P],
    "st_kmap_strided_query": [_P, _I, _L, _P, ctypes.POINTER(OutGeom), _L, _P, _L, _L, _P, _P, _P],
    "st_outcoords_brick_inverse": [_P, _I, _L, _P, ctypes.POINTER(OutGeom), _L, _L, _L, _P, _L, _P, _L, _P, _P, _P],
    "st_kmap_invert": [_P, _L, _L, _L, _I, _L, _P, _P, _P, _P, _P],
    "st_kmap_sort_workspace": [_L, ctypes.POINTER(ctypes.c_size_t)],
    "st_kmap_sort_rows": [_P, _I, _I, _L, _P, _P, _P, _P, ctypes.c_size_t, _P],
    "st_kmap_pairs_sizes": [_L, _I, ctypes.POINTER(_L)],
    "st_kmap_pairs": [_P, _L, _L, _L, _I, _L, _P, _L, _I, _P, _P, _P, _L, _P],
    "st_kmap_pairs_chunk_keys": [_P, _P, _P, _I, _I, _L, _L, _P, _P],
    "st_kmap_pairs_chunk_order": [_P, _P, _P, _I, _I, _L, _L, _P, _P],
    "st_kmap_plans_layout": [_L, _I, _I, _P],
    "st_kmap_plans": [_P, _L, _L, _P, _I, _L, _L, _I, _I, _P, _P, _P],
    "st_wgrad_pairs": [_P, _L, _P, _L, _P, _P, _P, _I, _I, _L, _P, _I, _I, _I, _P, _P, _I, _P],
    "st_weight_prep": [_P, _P, _I, _I, _I, _I, _I, _P],
    "st_tile_plan": [_P, _L, _L, _P, _I, _I, _P, _L, _L, _P, _P, _P, _P],
    "st_column_sum": [_P, _L, _I, _I, _P, _P, _I, _P],
    "st_column_sum_noalloc": [_P, _L, _I, _I, _P, _I, _P],
    "st_gather_gemm_tiled": [_P, _L, _P, _P, _P, _P, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P],
    "st_gather_gemm_tiled_epilogue": [_P, _L, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _L, _I, _I, _I, _I,
                                      _P],
    "st_gather_gemm": [_P, _L, _P, _L, _L, _P, _I, _P, _P, _P, _P, _L, _I, _I, _I, _I, _P],
    "st_wgrad": [_P, _L, _P, _P, _L, _L, _P, _L, _I, _I, _I, _I, _P, _L, _P, _I, _P],
    "st_hashfly_gemm": [_P, _L, _P, _I, _L, _P, ctypes.POINTER(Lookup), _P, _P, _L, _P, _P, _P, _I, _I, _I, _P],
    "st_to_dense": [_P, _L, _I, _I, _P, _I, _L, _L, _L, _L, _P, _P],
    "st_from_dense": [_P, _L, _L, _L, _L, _I, _I, _P, _I, _L, _P, _P],
    "st_mask_spatial_range": [_P, _I, _L, ctypes.POINTER(_L), _P, _P],
    "st_pool_workspace": [_L, ctypes.POINTER(ctypes.c_size_t)],
    "st_pool_plan": [_P, _I, _L, _I, _I, _I, _P, ctypes.c_size_t, _P, _P, _P, _P, _P, _P],
    "st_pool_forward": [_P, _I, _I, _P, _P, _L, _I, _P, _P],
    "st_pool_backward": [_P, _P, _P, _L, _I, _I, _P, _P, _I, _P, _P],
    "st_upsample": [_P, _P, _I, _L, _I, _I, _I, _P, _P, _P],
    "st_upsample_backward": [_P, _L, _I, _I, _I, _P, _P],
    "st_bn_workspace": [_L, _I, _I, ctypes.POINTER(_L)],
    "st_bn_forward": [_P, _L, _I, _I, _P, _I, _I, _P, _P, _P, _I, _I, ctypes.c_float, ctypes.c_float, _P, _P, _P,
                      _P, _P, _P, _L, _P, _P],
    "st_bn_backward": [_P, _P, _P, _L, _I, _I, _P, _I, _I, _P, _I, _I, _P, _P, _P, _P, _L, _P, _P, _P, _P, _P],
    "st_hashfly_wgrad": [_P, _L, _P, _P, _I, _L, _P, ctypes.POINTER(Lookup), _P, _P, _L, _I, _I, _I, _P, _L, _P,
                         _I, _P],
}
_RESTYPES = {"st_version": ctypes.c_char_p}

_lib = None


def lib_path() -> Path:
    return _LIB_PATH


def exported_symbols():
    """Names of the C entry points this binding declares."""
    return list(_SIGNATURES)


def lib():
    """Load (once) and return the ctypes handle of the HIP library."""
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        raise RuntimeError(
            f"sparsetriton_amd: HIP library not built ({_LIB_PATH} missing); "
            "run `python -c 'import __graft_entry__ as g; g.build()'` or `python sparsetriton_amd/_build.py`"
        )
    handle = ctypes.CDLL(str(_LIB_PATH), mode=os.RTLD_LOCAL | getattr(os, "RTLD_NOW", 2))
    for name, args in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != ST_OK:
        raise RuntimeError(f"sparsetriton_amd: {what} failed: {ERRORS.get(rc, rc)} ({rc})")


_FNS = {}


def call(name: str, *args) -> None:
    fn = _FNS.get(name)
    if fn is None:
        fn = _FNS[name] = getattr(lib(), name)
    rc = fn(*args)
    if rc != ST_OK:
        check(rc, name)


def ptr(t) -> int:
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    return t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device):
    """Raw hipStream_t of torch's current stream on `device` (the kernel launches are cheap
    enough that this lookup shows up in map builds, hence the direct binding)."""
    if _raw_stream is not None:
        idx = device.index
        return _raw_stream(idx if idx is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def require_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"sparsetriton_amd: {what} must live on the GPU (got {t.device}); "
            "the HIP kernels are the only implementation of this path"
        )


def coord_code(dtype: torch.dtype) -> int:
    try:
        return COORD_DTYPES[dtype]
    except KeyError:
        raise TypeError(f"unsupported coordinate dtype {dtype}; use int16, int32 or int64") from None


def feat_code(dtype: torch.dtype) -> int:
    try:
        return FEAT_DTYPES[dtype]
    except KeyError:
        raise TypeError(f"unsupported feature dtype {dtype}; use float32, float16 or bfloat16") from None


F32_BF16X3 = 3


def compute_code(dtype: torch.dtype) -> int:
    """dtype code for a GEMM entry point: fp32 follows ``config.get_fp32_precision()``."""
    code = feat_code(dtype)
    if code == 0:
        from sparsetriton_amd.config import get_fp32_precision

        if get_fp32_precision() == "bf16x3":
            return F32_BF16X3
    return code


def fill_(t: torch.Tensor, value: int) -> torch.Tensor:
    """Fill a 4- or 8-byte-element device tensor with a raw bit pattern via the library."""
    s = stream_of(t.device)
    n = t.numel()
    if t.element_size() == 8:
        call("st_fill_u64", ptr(t), n, ctypes.c_uint64(value & 0xFFFFFFFFFFFFFFFF), s)
    elif t.element_size() == 4:
        call("st_fill_u32", ptr(t), n, ctypes.c_uint32(value & 0xFFFFFFFF), s)
    else:
        raise TypeError("fill_ needs 4- or 8-byte elements")
    return t
