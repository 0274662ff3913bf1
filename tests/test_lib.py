"""The C-ABI library: it loads, and exports every entry point include/*.h declares (no GPU calls)."""

import ctypes
import re
from pathlib import Path

import torch

from sparsetriton_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        names |= set(re.findall(r"^\s*(?:int|const char\*|size_t|void)\s+(st_\w+)\s*\(", text, re.M))
    return names


def test_header_declares_entry_points():
    names = _declared()
    assert {"st_hash_insert", "st_hash_query", "st_kmap_query", "st_outcoords_plan", "st_outcoords_emit",
            "st_gather_gemm", "st_wgrad", "st_hashfly_gemm", "st_hashfly_wgrad"} <= names


def test_library_exports_every_declared_symbol():
    handle = ctypes.CDLL(str(_lib.lib_path()))
    missing = [n for n in sorted(_declared()) if not hasattr(handle, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_header():
    assert set(_lib.exported_symbols()) == _declared()


def test_version_and_arg_checks():
    lib = _lib.lib()
    assert lib.st_version().startswith(b"sparsetriton_amd")
    # argument validation runs on the host: no device memory is touched
    assert lib.st_hash_insert(None, 0, 5, 1, None, None, 10, None, None) == -1
    assert lib.st_gather_gemm(None, 0, None, 0, 0, None, 1, None, None, None, None, 0, 0, 8, 8, 0, None) == -1
    assert lib.st_weight_prep(None, None, 27, 4, 4, 0, 0, None) == -1


def test_plan_layout_with_an_automatic_chunk_size():
    """st_kmap_plans_layout is host arithmetic: a pair list cut at ST_PAIR_CHUNK_AUTO (-1) is
    bounded by min(2048 + K, K * n / 1024 + K) chunks and keeps K + 2 cstart words."""
    lib = _lib.lib()
    L = (ctypes.c_int64 * 12)()
    for n, K in ((100, 27), (5000, 27), (1_000_000, 27), (300_000, 125)):
        assert lib.st_kmap_plans_layout(n, K, -1, L) == 0
        assert L[11] == min(2048 + K, K * n // 1024 + K)
        assert L[7] - L[6] >= 4 * (K + 2)  # cstart region (ends at the chunk order)
        assert lib.st_kmap_plans_layout(n, K, 2048, L) == 0
        assert L[11] == K * n // 2048 + K
    assert lib.st_kmap_plans_layout(100, 27, -2, L) == -1


def test_subm_fly_eligibility_is_size_aware():
    """st_subm_fly_ok(n, Kd, Nd, K, dtype) is host arithmetic: the brick-index gather takes n rows
    only while n * Kd * element size stays under 2^31 - 64 bytes (its 32-bit buffer offsets), so a
    convolution over more rows goes to the table-probing kernels instead of failing in the call."""
    import torch

    from sparsetriton_amd.nn.functional.conv.funcs.implicit_hashfly_gemm import subm_fly_ok

    lib = _lib.lib()
    lim = (1 << 31) - 64
    for code, esz in ((3, 4), (2, 2), (1, 2)):
        for kd in (64, 128):
            n_max = (lim - 1) // (kd * esz)  # largest n with n * kd * esz < lim
            assert lib.st_subm_fly_ok(n_max, kd, 64, 27, code) == 1
            assert lib.st_subm_fly_ok(n_max + 1, kd, 64, 27, code) == 0
    assert lib.st_subm_fly_ok(-1, 64, 64, 27, 2) == 0
    assert lib.st_subm_fly_ok(1000, 64, 64, 27, 0) == 0  # IEEE fp32: not built
    assert lib.st_subm_fly_ok(1000, 128, 128, 27, 3) == 0  # split fp32 at 128 x 128: not built
    # the Python predicate checks both directions: with C_out > C_in the input gradient's
    # operand (n x C_out) is the larger one
    n_fwd_only = (lim - 1) // (64 * 2)  # fits n x 64 bf16 but not n x 128
    assert lib.st_subm_fly_ok(n_fwd_only, 64, 128, 27, 2) == 1
    assert not subm_fly_ok(n_fwd_only, 64, 128, 27, torch.bfloat16)
    assert subm_fly_ok((lim - 1) // (128 * 2), 64, 128, 27, torch.bfloat16)


def test_fly_gemm_and_masks_query_argument_checks():
    """Host-side checks of the brick-index entry points (no device memory is touched): the fly
    GEMM takes only ST_GATHER_REVERSE_K as a flag, and a subm query needs a map or mask output."""
    lib = _lib.lib()
    nbytes = ctypes.c_int64()
    assert lib.st_kmap_subm_workspace(0, 1, 8, 8, 8, ctypes.byref(nbytes)) == 0
    bad_flags = _lib.GATHER_REVERSE_K << 1
    # n = 0: returns before any launch once the arguments are valid
    args = (None, None, _lib.coord_code(torch.int16), 0, None, 27, 1, 8, 8, 8, None, nbytes.value, None, None, None,
            None, 64, 64, _lib.compute_code(torch.bfloat16))
    assert lib.st_subm_fly_gemm(*args, 0, None) == 0
    assert lib.st_subm_fly_gemm(*args, _lib.GATHER_REVERSE_K, None) == 0
    assert lib.st_subm_fly_gemm(*args, bad_flags, None) == -1
    # one row, neither nbr nor row_masks: rejected before the launch
    assert lib.st_kmap_subm_workspace(1, 1, 8, 8, 8, ctypes.byref(nbytes)) == 0
    assert lib.st_kmap_subm_query(ctypes.c_void_p(16), _lib.coord_code(torch.int16), 1, ctypes.c_void_p(16), 27, 1, 8, 8,
                                  8, ctypes.c_void_p(16), nbytes.value, None, None, None) == -1
