"""The measurement helper behind bench.py's measured peaks (``st_mfma_peak``): its operation
count is the launch geometry's, its outputs are finite, and the rate it gives is a plausible
share of the published dense bf16 MFMA peak (2.5 PFLOP/s)."""
import ctypes

import pytest
import torch

from sparsetriton_amd import _lib

pytestmark = pytest.mark.gpu


def test_mfma_peak_counts_and_rate():
    dev = torch.device("cuda:0")
    blocks, iters = 2 * torch.cuda.get_device_properties(dev).multi_processor_count, 400
    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    flops = ctypes.c_int64()
    stream = _lib.stream_of(dev)
    _lib.call("st_mfma_peak", iters, blocks, _lib.ptr(out), ctypes.byref(flops), stream)
    torch.cuda.synchronize()
    assert flops.value == blocks * 4 * iters * 8 * 2 * 16 * 16 * 32
    assert bool(torch.isfinite(out).all())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        _lib.call("st_mfma_peak", iters, blocks, _lib.ptr(out), ctypes.byref(flops), stream)
    e1.record()
    e1.synchronize()
    tflops = 3 * flops.value / (e0.elapsed_time(e1) * 1e-3) / 1e12
    assert 250.0 < tflops < 2750.0, tflops


def test_mfma_peak_rejects_bad_arguments():
    flops = ctypes.c_int64()
    lib = _lib.lib()
    assert lib.st_mfma_peak(0, 1, None, ctypes.byref(flops), None) != 0
    assert lib.st_mfma_peak(10, 1, None, ctypes.byref(flops), None) != 0
