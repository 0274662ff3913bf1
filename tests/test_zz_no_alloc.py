"""st_column_sum_noalloc (no reference counterpart; for callers that cannot allocate) against
st_column_sum through the C ABI: bit-identical sums on two calls in a row, the second smaller, so
the shared device array's leftovers from the first call cannot leak into the second."""

import pytest
import torch

from sparsetriton_amd import _lib

pytestmark = pytest.mark.gpu


def _with_workspace(Y, out_dtype):
    n, C = Y.shape
    partials = torch.empty((1024 * C,), dtype=torch.float32, device=Y.device)
    out = torch.empty((C,), dtype=out_dtype, device=Y.device)
    _lib.call("st_column_sum", _lib.ptr(Y), n, C, _lib.feat_code(Y.dtype), _lib.ptr(partials), _lib.ptr(out),
              _lib.feat_code(out_dtype), _lib.stream_of(Y.device))
    return out


def _no_alloc(Y, out):
    n, C = Y.shape
    _lib.call("st_column_sum_noalloc", _lib.ptr(Y), n, C, _lib.feat_code(Y.dtype), _lib.ptr(out),
              _lib.feat_code(out.dtype), _lib.stream_of(Y.device))
    return out


@pytest.mark.parametrize("dtype,out_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.float32),
                                             (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16)])
@pytest.mark.parametrize("first,second", [((470_532, 64), (3001, 64)), ((200_000, 2048), (50, 300)),
                                          ((5000, 7), (1, 7)), ((100_000, 128), (0, 128))])
def test_noalloc_matches_workspace_entry_point(device, dtype, out_dtype, first, second):
    g = torch.Generator(device="cpu").manual_seed(first[0] + first[1])
    for n, C in (first, second):
        Y = torch.randn((n, C), generator=g).to(device, dtype)
        ref = _with_workspace(Y, out_dtype)
        out = torch.full((C,), float("nan"), dtype=out_dtype, device=device)
        got = _no_alloc(Y, out)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (n, C)
        exact = Y.double().sum(0) if n else torch.zeros(C, dtype=torch.float64, device=device)
        tol = (4e-3 if out_dtype != torch.float32 else 1e-5) * max(1.0, n ** 0.5) * 4
        assert (got.double() - exact).abs().max().item() <= tol


def test_noalloc_rejects_oversized_columns(device):
    C = _lib.COLUMN_SUM_NOALLOC_MAX_C + 1
    Y = torch.zeros((4, C), device=device)
    out = torch.zeros((C,), device=device)
    with pytest.raises(RuntimeError, match="invalid argument"):
        _no_alloc(Y, out)


def test_noalloc_allocates_nothing(device):
    """Repeated calls leave torch's allocator untouched (the library does not allocate either:
    its partials live in the static device array)."""
    Y = torch.randn((300_000, 64), device=device)
    out = torch.empty((64,), device=device)
    _no_alloc(Y, out)
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats(device)["allocation.all.allocated"]
    for _ in range(5):
        _no_alloc(Y, out)
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats(device)["allocation.all.allocated"] == before
    assert torch.equal(out, _with_workspace(Y, torch.float32))
