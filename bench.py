#!/usr/bin/env python
"""Benchmark: SubMConv3D k3 64->64 forward + backward on one MI355X (headline configuration 2).

Workload: the seeded LiDAR-like voxel set of config 2 (B=4, 1440x1440x41,
~118k voxels per sample), SubMConv3D 64->64, kernel 3, synthetic N(0,1)
features and output gradients, weights U(+-1/sqrt(64*27)).  Inputs are resident
in HBM before timing starts.

A step = one forward + backward (input and weight gradient) of the layer
through the public API (``sparse_conv3d`` + autograd), with the kernel map
already cached on the tensor -- as in a stack of submanifold layers, where it
is built once per coordinate set.  The kernel-map build (the coordinates' brick
index + neighbour query, mask-sorted tile plan, pair list) is timed separately and reported as
``kmap_build_ms``.  Before each timed measurement the same work runs back to back, untimed,
for ``SETTLE_MS`` of wall time (``clock_settle`` in the JSON line): the GPU's clocks ramp up
under sustained load, and without it the timed window ran 6-10 % below the steady state.

value = effective TFLOP/s = 6 * P * C_in * C_out / step time, P = exact number
of (input, output, offset) pairs.  ``roofline`` covers the dominant kernel,
timed with HIP events on the stream it runs on.  ``cpu_baseline`` times the
reference algorithm's CPU port (oracle/st_oracle.c: 31-bit hash with 128-probe
cap, output-major map, output-stationary forward, scatter input gradient, weight
gradient by row slabs x offsets as the reference's grid; fp32, OpenMP) on the same voxel set.

``measured_peaks`` confirms the spec-sheet peaks on the box: a 1 GiB device-to-device copy and
the dense bf16 MFMA rate of register-only MFMA chains (``st_mfma_peak``); every roofline also
gives its achieved rate as ``frac_of_measured_peak`` of the measured rate for its bound (``frac``
stays against the published peak).

The default run also measures the other benchmark configurations -- config 2 in bf16, the
strided (config 3) and transposed (config 4) convolutions, the 1M-voxel layer (config 5) with
either algorithm -- into ``configs``: one record each with its step time, effective TFLOP/s, the
three GEMM kernels timed alone and the roofline of the dominant one (``--no-configs`` skips them).

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--dtype f32|bf16] [--no-cpu]
                       [--fp32-precision bf16x3|ieee] [--profile] [--no-configs]
                       [--workload config2|config3|...]

``--workload`` other than config2 measures one other benchmark configuration on its own: one
JSON line with the same fields, the step timed the same way, plus the first-call time (map build
+ forward).
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"hbm_GBps": 8000.0, "f32_TFLOPs": 157.3, "bf16_TFLOPs": 2500.0, "f16_TFLOPs": 2500.0}
METRIC = "SubMConv3D k3 fwd+bwd effective TFLOP/s + kernel-map build ms, 1 MI355X"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


SETTLE_MS = 60.0  # untimed back-to-back work before each timed GPU measurement


def _settle(torch, fn, ms=SETTLE_MS):
    """Run fn back to back for `ms` of wall time, untimed, and return the call count.  The GPU's
    clocks ramp up under sustained load: a window timed right after the host's map builds and
    data uploads ran 6-10 % slower than the steady state (config 2 fp32: 0.427 ms a step after 10
    warm-up steps, 0.403 ms after 100 or 300; bf16 0.189 vs 0.171 ms).  A synchronisation every 16
    calls keeps the host from queueing far ahead, so the wall time is GPU time."""
    fn()  # (a first call may include one-time set-up: the clock starts after it)
    torch.cuda.synchronize()
    t0, n = time.perf_counter(), 1
    while (time.perf_counter() - t0) * 1e3 < ms:
        fn()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def _events(torch, fn, reps):
    """Per-call durations (ms) of fn() with HIP events on the current stream."""
    times = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    return np.array(times)


def _events_batch(torch, fn, reps):
    """Average device time (ms) of fn() over reps back-to-back calls, bracketed by HIP events
    on the current stream (the stream every kernel here is launched on); the host's launch
    work overlaps the previous call's kernels, so this is the kernels' time, not the host's."""
    fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_config2_subm64.md")
# the sources of the gather and weight-gradient kernels whose counters the traffic file holds
GEMM_SOURCES = ("gemm_kernels.h", "gemm_wide.h", "gemm_x3.h", "gemm_x3.hip", "mfma.h", "nbr_src.h")


def gemm_sources_sha():
    """sha256 (16 hex digits) over the GEMM kernel sources, in GEMM_SOURCES order: the key that ties
    a traffic measurement to the kernels it measured."""
    import hashlib

    h = hashlib.sha256()
    for name in GEMM_SOURCES:
        with open(os.path.join(ROOT, "sparsetriton_amd", "csrc", name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read() + b"\0")
    return h.hexdigest()[:16]


def _measured_traffic(dtype, role):
    """(HBM bytes per launch of a GEMM role, provenance) from the committed rocprofv3 counter summary
    (lines `traffic <dtype> <role> <bytes>`, `measured_commit <sha>`, `gemm_sources_sha <sha>`).
    The bytes are None when the file has no entry or when the GEMM sources have changed since the
    counters were taken (the figure would describe other kernels)."""
    src = {"file": os.path.relpath(TRAFFIC_FILE, ROOT), "measured_commit": None, "gemm_sources_sha": None,
           "current_gemm_sources_sha": gemm_sources_sha(), "stale": None}
    val = None
    try:
        for line in open(TRAFFIC_FILE):
            f = line.split()
            if len(f) == 4 and f[0] == "traffic" and f[1] == dtype and f[2] == role:
                val = float(f[3])
            elif len(f) == 2 and f[0] in ("measured_commit", "gemm_sources_sha"):
                src[f[0]] = f[1]
    except OSError:
        pass
    src["stale"] = src["gemm_sources_sha"] != src["current_gemm_sources_sha"]
    return (None if src["stale"] else val), src


def gemm_roofline(kernel, kernel_ms, n_in, n_out, cin, cout, K, P, dts, fp32_precision, traffic=None,
                  traffic_source=None):
    """Roofline of one gather-GEMM / weight-gradient launch.  Algorithmic work: 2 P C_in C_out flops;
    bytes = s (N_in C_in + N_out C_out + K C_in C_out) + 8 P (the two feature arrays once, the weights,
    one int32 (in, out) index pair per map pair; s = element size).  The binding roof is HBM when the
    intensity lies below the ridge point of the arithmetic the kernel runs (split fp32: a third of
    the bf16 peak, three bf16 products per fp32 product), else the MFMA peak."""
    gemm_flops = 2.0 * P * cin * cout
    esz = 4 if dts == "f32" else 2
    gemm_bytes = esz * (n_in * cin + n_out * cout + K * cin * cout) + 8 * P
    if dts == "f32" and fp32_precision == "bf16x3":
        mfma_peak = PEAK["bf16_TFLOPs"] / 3.0
        note = "dense bf16 MFMA peak / 3 (three bf16 products per fp32 product)"
    elif dts == "f32":
        mfma_peak, note = PEAK["f32_TFLOPs"], "dense f32 MFMA peak"
    else:
        mfma_peak, note = PEAK["bf16_TFLOPs"], f"dense {dts} MFMA peak"
    tflops = gemm_flops / (kernel_ms * 1e-3) / 1e12
    intensity = gemm_flops / gemm_bytes
    ridge = mfma_peak * 1e12 / (PEAK["hbm_GBps"] * 1e9)
    common = {"traffic": traffic, "traffic_unit": "bytes/launch", "traffic_source": traffic_source,
              "kernel": kernel, "kernel_avg_ms": kernel_ms, "algorithmic_bytes_per_launch": gemm_bytes,
              "algorithmic_flops_per_launch": gemm_flops, "flops_per_byte": intensity, "ridge_flops_per_byte": ridge,
              "mfma_TFLOPs": tflops, "mfma_peak_TFLOPs": mfma_peak, "mfma_frac": tflops / mfma_peak,
              "mfma_peak_note": note}
    if intensity < ridge:
        gbps = gemm_bytes / (kernel_ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": gbps, "peak": PEAK["hbm_GBps"], "unit": "GB/s",
                "frac": gbps / PEAK["hbm_GBps"], **common}
    return {"bound": "mfma", "achieved": tflops, "peak": mfma_peak, "unit": "TFLOP/s", "frac": tflops / mfma_peak,
            **common}


def measured_peaks(torch, dev):
    """The chip's sustained rates, measured on the box beside the spec-sheet peaks the rooflines
    use: HBM as a 1 GiB device-to-device copy (bytes read + written / time, 5 back-to-back copies
    after 2 untimed), dense bf16 MFMA as `st_mfma_peak` (8 independent 16x16x32 chains per wave on
    register operands, four workgroups of four waves per CU; 3 launches after 1 untimed)."""
    import ctypes

    from sparsetriton_amd import _lib

    n = 1 << 28  # fp32 elements: 1 GiB
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    reps = 5
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    e1.synchronize()
    copy_gbps = 2 * 4 * n * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    blocks, iters, launches = 4 * cus, 500, 3
    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    flops = ctypes.c_int64()
    stream = _lib.stream_of(dev)
    _lib.call("st_mfma_peak", iters, blocks, _lib.ptr(out), ctypes.byref(flops), stream)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(launches):
        _lib.call("st_mfma_peak", iters, blocks, _lib.ptr(out), ctypes.byref(flops), stream)
    e1.record()
    e1.synchronize()
    bf16 = flops.value * launches / (e0.elapsed_time(e1) * 1e-3) / 1e12
    torch.cuda.empty_cache()
    return {"hbm_copy_GBps": copy_gbps, "bf16_mfma_TFLOPs": bf16, "split_fp32_mfma_TFLOPs": bf16 / 3.0,
            "spec": dict(PEAK), "copy": "1 GiB device-to-device, 2 x 1 GiB moved per copy",
            "mfma": f"st_mfma_peak: {blocks} workgroups x 4 waves x {iters} x 8 chains of 16x16x32 bf16"}


def with_measured_peak(roof, peaks):
    """The roofline's achieved rate also as a fraction of the rate measured on the box for its
    bound (copy bandwidth, or the MFMA rate scaled like the spec peak it uses)."""
    if not roof or not peaks:
        return roof
    if roof["bound"] == "hbm":
        m = peaks["hbm_copy_GBps"]
    else:
        m = peaks["bf16_mfma_TFLOPs"] * roof["mfma_peak_TFLOPs"] / PEAK["bf16_TFLOPs"]
    roof["measured_peak"] = m
    roof["frac_of_measured_peak"] = roof["achieved"] / m
    return roof


def _stats(t):
    return {"median": float(np.median(t)), "p10": float(np.percentile(t, 10)), "p90": float(np.percentile(t, 90))}


def _port_pass(O, coords, shape, X, W, dY):
    """One pass of the reference-algorithm port: its hash + map build, fwd, dgrad, wgrad (seconds)."""
    off = O.target_offsets(3, 1, 1, False)
    t0 = time.perf_counter()
    h = O.RefHash(coords)
    nbr = h.kmap(coords, off, 1, shape)
    t1 = time.perf_counter()
    O.ref_fwd_f32(X, W, nbr)
    t2 = time.perf_counter()
    O.ref_dgrad_f32(dY, W, nbr, coords.shape[0])
    t3 = time.perf_counter()
    O.ref_wgrad_f32(X, dY, nbr, W.shape[0])
    t4 = time.perf_counter()
    return (t1 - t0, t2 - t1, t3 - t2, t4 - t3), int((nbr >= 0).sum()), h.dropped


def _port_timed(O, threads, coords, shape, X, W, dY, warmup, iters, budget_s=None):
    """Median / p10 / p90 (ms) of each stage over `iters` timed passes after `warmup`, on `threads`
    OpenMP threads (stops early once `budget_s` seconds of timed passes are spent)."""
    O.set_threads(threads)
    for _ in range(warmup):
        _port_pass(O, coords, shape, X, W, dY)
    rows, P, dropped = [], 0, 0
    t_start = time.perf_counter()
    for _ in range(iters):
        t, P, dropped = _port_pass(O, coords, shape, X, W, dY)
        rows.append(t)
        if budget_s is not None and time.perf_counter() - t_start > budget_s:
            break
    a = np.array(rows) * 1e3
    gemm = a[:, 1] + a[:, 2] + a[:, 3]
    flops = 6.0 * P * X.shape[1] * W.shape[2]
    gflops = flops / (gemm * 1e-3) / 1e9
    return {"threads": threads, "iters": len(rows), "warmup": warmup, "pairs": P, "inserts_dropped": dropped,
            "kmap_build_ms": _stats(a[:, 0]), "fwd_ms": _stats(a[:, 1]), "dgrad_ms": _stats(a[:, 2]),
            "wgrad_ms": _stats(a[:, 3]), "fwd_bwd_GFLOPs": _stats(gflops)}


def config1_inputs(seed=0):
    """SubMConv3D 16->32 on 4096 uniform voxels in 2 x 64^3, X ~ N(0,1), dY ~ N(0,1),
    W ~ U(+-1/sqrt(16*27))."""
    from sparsetriton_amd import workloads

    coords, shape = workloads.config1(seed=seed)
    rng = np.random.default_rng(seed + 1)
    X = rng.standard_normal((coords.shape[0], 16)).astype(np.float32)
    bound = 1.0 / np.sqrt(16 * 27)
    W = rng.uniform(-bound, bound, (27, 16, 32)).astype(np.float32)
    dY = rng.standard_normal((coords.shape[0], 32)).astype(np.float32)
    return coords, shape, X, W, dY


def cpu_baseline(coords, shape, X, W, dY, profile=False):
    """The reference algorithm's CPU port (oracle/st_oracle.c ref_*: 31-bit key2 table with the
    128-probe cap, output-major map, output-stationary forward, scatter input gradient, row-slab x offset
    weight gradient; fp32, OpenMP), as planned for the CPU baseline: config 1 with >= 10 warmup and
    >= 50 timed passes on all host threads and on one, and beside it a bounded sample of the
    benchmark workload itself (config 2) on all host threads -- its figure is `value`."""
    from oracle import oracle as O

    all_threads = O.num_threads()
    c1 = config1_inputs()
    iters1 = 5 if profile else 50
    cfg1 = {"all": _port_timed(O, all_threads, *c1, warmup=2 if profile else 10, iters=iters1),
            "one": _port_timed(O, 1, *c1, warmup=2 if profile else 10, iters=iters1)}
    cfg2 = _port_timed(O, all_threads, coords, shape, X, W, dY, warmup=1, iters=1 if profile else 20,
                       budget_s=20.0)
    O.set_threads(all_threads)
    P = cfg2["pairs"]
    gemm_ms = cfg2["fwd_ms"]["median"] + cfg2["dgrad_ms"]["median"] + cfg2["wgrad_ms"]["median"]
    return {
        "value": 6.0 * P * X.shape[1] * W.shape[2] / (gemm_ms * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "cores": all_threads,
        "kind": "port",
        "sample": (f"config-2 voxel set (N={coords.shape[0]}), fwd+dgrad+wgrad in fp32 over the reference-hash "
                   f"kernel map ({P} pairs, {cfg2['inserts_dropped']} inserts dropped by the 128-probe cap); "
                   f"median of {cfg2['iters']} passes after 1 warmup on {all_threads} OpenMP threads"),
        "os_cpu_count": os.cpu_count(),
        "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"),
        "config2": cfg2,
        "config1": cfg1,
    }


def gpu_config1(torch, reps):
    """BASELINE config 1 on the GPU in the same run as the CPU baseline: the layer's kernel-map build
    (new coordinate set + forward) and its fwd+bwd step with the map cached, fp32."""
    from sparsetriton_amd import SparseTensor
    from sparsetriton_amd.nn.functional import sparse_conv3d

    coords, shape, X, W, dY = config1_inputs()
    dev = torch.device("cuda:0")
    c = torch.as_tensor(coords, device=dev).to(torch.int16)
    x = torch.as_tensor(X, device=dev)
    w = torch.as_tensor(W, device=dev).requires_grad_(True)
    g = torch.as_tensor(dY, device=dev)

    def first():
        sp = SparseTensor(x.clone().requires_grad_(True), c, spatial_shape=shape, batch_size=2)
        return sp, sparse_conv3d(sp, w, 3)

    sp, out = first()
    feats = sp.F

    def step():
        feats.grad = None
        w.grad = None
        sparse_conv3d(sp, w, 3).F.backward(g)

    for _ in range(10):
        step()
    first_t = _events(torch, lambda: first(), reps)
    step_t = _events(torch, step, reps)
    km = sp._cache.neighbor_indices[(3, 1, 1, 1, True, False)][1]
    P = km.num_pairs()
    return {"workload": "config1: SubMConv3D 16->32 k3, B=2, 64^3, 4096 uniform voxels, fp32", "pairs": P,
            "first_call_build_plus_fwd_ms": _stats(first_t), "fwd_bwd_step_ms": _stats(step_t),
            "fwd_bwd_GFLOPs": 6.0 * P * 16 * 32 / (np.median(step_t) * 1e-3) / 1e9}


EXTRA = {
    # name: (description, C_in, C_out, k, stride, padding, transposed, submanifold, dtype, algorithm)
    "config2-bf16": ("SubMConv3D 64->64 k3 in bf16 on the config-2 voxel set", 64, 64, 3, 1, 1, False, True,
                     "bf16", "precomputed"),
    "config3": ("SparseConv3D 64->128 k3 s2 p1 on the config-2 voxel set", 64, 128, 3, 2, 1, False, False, "f32",
                "precomputed"),
    "config4": ("SparseConvTransposed3D 128->64 k3 s2 p1 on config 3's output coordinates", 128, 64, 3, 2, 1, True,
                False, "bf16", "precomputed"),
    "config5": ("SubMConv3D 128->128 k3, 1M voxels of 2-voxel walls in 256^3 (PrecomputedNeighborGEMM)", 128, 128,
                3, 1, 1, False, True, "bf16", "precomputed"),
    "config5-hashfly": ("SubMConv3D 128->128 k3, same set (ImplicitHashFlyGEMM)", 128, 128, 3, 1, 1, False, True,
                        "bf16", "hashfly"),
    "config2-bias": ("SubMConv3D 64->64 k3 with bias (the module default), config-2 set", 64, 64, 3, 1, 1, False,
                     True, "f32", "precomputed"),
}
WITH_BIAS = {"config2-bias"}
# the configurations measured beside the headline in the default run (one record each)
DEFAULT_CONFIGS = ("config2-bf16", "config3", "config4", "config5", "config5-hashfly")


def measure_extra(name, steps, warmup, profile=False, fp32_precision="bf16x3", coords_cache=None):
    """One benchmark configuration other than the headline one, as a record: the layer's fwd+bwd
    step (map cached) through sparse_conv3d and autograd, timed like the headline, its first call
    (map build + forward), the three GEMM kernels timed alone with HIP events on the launch stream
    (forward gather, input-gradient gather, weight gradient with its reduce; for hash-fly the
    forward is the in-GEMM-lookup gather) and the roofline of the dominant one.  ``coords_cache``
    (a dict) keeps the seeded voxel sets across calls."""
    import torch

    from sparsetriton_amd import SparseTensor, _lib, workloads
    from sparsetriton_amd.config import ConvAlgo, get_conv_algo, set_conv_algo, set_fp32_precision
    from sparsetriton_amd.nn.functional import sparse_conv3d
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import (
        gather_gemm_dgrad,
        gather_gemm_fwd,
        weight_gradient,
        weight_prep,
    )

    desc, Cin, Cout, k, s, p, tr, subm, dts, algo = EXTRA[name]
    prev_algo = get_conv_algo()
    set_fp32_precision(fp32_precision)
    set_conv_algo(ConvAlgo.ImplicitHashFlyGEMM if algo == "hashfly" else ConvAlgo.PrecomputedNeighborGEMM)
    dev = torch.device("cuda:0")
    dtype = {"f32": torch.float32, "bf16": torch.bfloat16}[dts]
    seed = 0
    cache = coords_cache if coords_cache is not None else {}
    setname = "config5" if name.startswith("config5") else "config2"
    if setname not in cache:
        cache[setname] = workloads.config5(seed=seed) if setname == "config5" else workloads.config2(seed=seed)
    coords_np, shape = cache[setname]
    batch = 1 if setname == "config5" else 4
    coords = torch.as_tensor(coords_np, device=dev).to(torch.int16)
    if name == "config4":
        # input = the output coordinates of config 3's strided convolution
        from sparsetriton_amd.nn.functional.conv.kmap import build_out_coords
        coords, shape, _ = build_out_coords(coords, shape, 3, stride=2, padding=1, submanifold=False)
        shape = tuple(int(v) for v in shape)
    N = coords.shape[0]
    g = torch.Generator(device="cpu").manual_seed(seed)
    X = torch.randn(N, Cin, generator=g).to(dev, dtype)
    bound = 1.0 / np.sqrt(Cin * k ** 3)
    W = ((torch.rand(k ** 3, Cin, Cout, generator=g) * 2 - 1) * bound).to(dev, dtype).requires_grad_(True)
    b = None
    if name in WITH_BIAS:
        b = ((torch.rand(Cout, generator=g) * 2 - 1) * bound).to(dev, dtype).requires_grad_(True)

    def fresh():
        feats = X.clone().requires_grad_(True)
        return feats, SparseTensor(feats, coords, spatial_shape=shape, batch_size=batch)

    def build():
        # a new coordinate set: table, kernel map (or hash-fly lookups) and all plans
        feats, sp = fresh()
        out = sparse_conv3d(sp, W, k, bias=b, stride=s, padding=p, transposed=tr, submanifold=subm)
        return sp, out

    # map build = first call's extra time over a cached call, both fwd only
    sp, out = build()
    torch.cuda.synchronize()
    n_out = out.F.shape[0]
    km = None
    if algo == "hashfly":
        P = None
    else:
        km = next(iter(sp._cache.neighbor_indices.values()))[1]
        km.prepare()
        P = km.num_pairs()
    dY = torch.randn(n_out, Cout, generator=g).to(dev, dtype)
    R = 3 if profile else 10
    settled = {"ms": SETTLE_MS, "calls_before_first_call_timing": _settle(torch, build)}
    build_t = _events(torch, build, R)

    feats = sp.F

    def step():
        feats.grad = None
        W.grad = None
        if b is not None:
            b.grad = None
        o = sparse_conv3d(sp, W, k, bias=b, stride=s, padding=p, transposed=tr, submanifold=subm)
        o.F.backward(dY)

    settled["steps_before_step_timing"] = _settle(torch, step)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps

    # the GEMM kernels alone (HIP events on the launch stream, back to back)
    KR = 5 if profile else 20
    Wd = W.detach()
    wt = weight_prep(Wd.contiguous(), _lib.W_TRANSPOSE)
    if algo == "hashfly":
        from sparsetriton_amd.nn.functional.conv.funcs.implicit_hashfly_gemm import fly_tile_order, subm_fly_gemm
        from sparsetriton_amd.nn.functional.conv.kmap import _offsets_i32, _target_offsets

        index = next(v for key, v in sp._cache.kmaps.items() if key[0] == "brick_index")
        offs = _offsets_i32(_target_offsets(k, 1, p, False, dev))
        order = fly_tile_order(index, offs, (k, 1, p))  # the step's cached order
        Wc = Wd.contiguous()
        kern = {"gather_fly_fwd": _events_batch(torch, lambda: subm_fly_gemm(X, index, offs, wt, order), KR),
                "gather_fly_dgrad": _events_batch(
                    torch, lambda: subm_fly_gemm(dY, index, offs, Wc, order, reverse_k=True), KR)}
        set_conv_algo(ConvAlgo.PrecomputedNeighborGEMM)  # an exact map of the same geometry: P and wgrad
        _, sp2 = fresh()
        sparse_conv3d(sp2, W, k, stride=s, padding=p, transposed=tr, submanifold=subm)
        km = next(iter(sp2._cache.neighbor_indices.values()))[1]
        km.prepare()
        P = km.num_pairs()
        kern["wgrad(+reduce)"] = _events_batch(torch, lambda: weight_gradient(X, dY, km, Wd.dtype), KR)
    else:
        kern = {"gather_gemm_fwd": _events_batch(torch, lambda: gather_gemm_fwd(X, km, wt), KR),
                "gather_gemm_dgrad": _events_batch(torch, lambda: gather_gemm_dgrad(dY, km, Wd.contiguous()), KR),
                "wgrad(+reduce)": _events_batch(torch, lambda: weight_gradient(X, dY, km, Wd.dtype), KR)}
    set_conv_algo(prev_algo)
    dom = max(kern, key=kern.get)
    # the input gradient reads dY (N_out x C_out) and writes dX: the same bytes as the forward
    roof = gemm_roofline(dom, kern[dom], N, n_out, Cin, Cout, k ** 3, P, dts, fp32_precision)
    value = 6.0 * P * Cin * Cout / (ms * 1e-3) / 1e12
    log(f"{name}: N_in={N} N_out={n_out} P={P}; step {ms:.3f} ms -> {value:.2f} TFLOP/s; "
        f"first-call (map build + fwd) median {np.median(build_t):.3f} ms; kernels {kern}; "
        f"roofline {dom}: {roof['frac'] * 100:.1f}% of the {roof['bound']} peak")
    return {
        "workload": f"{name}: {desc}", "dtype": dts, "fp32_precision": fp32_precision if dts == "f32" else None,
        "algorithm": algo, "voxels_in": N, "voxels_out": n_out, "pairs": P, "C_in": Cin, "C_out": Cout,
        "seed": seed, "steps": steps, "warmup": warmup, "clock_settle": settled, "ms_per_step": ms,
        "effective_TFLOPs": value, "first_call_build_plus_fwd_ms": _stats(build_t), "kernels_avg_ms": kern,
        "roofline": roof,
    }


def run_extra(args):
    """One JSON line for a benchmark configuration other than the headline one (measure_extra)."""
    rec = measure_extra(args.workload, args.steps, args.warmup, args.profile, args.fp32_precision)
    line = {
        "metric": METRIC, "value": rec["effective_TFLOPs"], "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "clock_settle": rec["clock_settle"], "ms_per_step": rec["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": rec["dtype"],
        "fp32_precision": rec["fp32_precision"], "data": "synthetic (seeded voxel set, N(0,1) features)",
        "config": {k: rec[k] for k in ("workload", "voxels_in", "voxels_out", "pairs", "C_in", "C_out", "seed",
                                       "algorithm")},
        "first_call_build_plus_fwd_ms": rec["first_call_build_plus_fwd_ms"],
        "kernels_avg_ms": rec["kernels_avg_ms"], "roofline": rec["roofline"],
    }
    print(json.dumps(line), flush=True)


def run_spatial(args):
    """The section-8(f) ops beside the convolution -- pooling and upsampling (reference
    nn/functional/spatial.py:26-535) and to_dense (utils/to_dense.py:30-282) -- on the config-2 voxel
    set with 64 channels: each op's HIP kernels timed with events (after the clock settle) against
    their algorithmic bytes and the HBM peak, one JSON line.  value = all ops' bytes over all ops'
    time."""
    import ctypes

    import torch

    from sparsetriton_amd import SparseTensor, _lib, workloads
    from sparsetriton_amd.nn.functional import sparse_pooling
    from sparsetriton_amd.utils.to_dense import to_dense

    dev = torch.device("cuda:0")
    dtype = {"f32": torch.float32, "bf16": torch.bfloat16}[args.dtype]
    esz = 4 if args.dtype == "f32" else 2
    fc = _lib.feat_code(dtype)
    C = 64
    g = torch.Generator().manual_seed(0)
    coords_np, shape = workloads.config2(seed=0)
    N = coords_np.shape[0]
    coords = torch.as_tensor(coords_np, device=dev).to(torch.int16)
    X = torch.randn(N, C, generator=g).to(dev, dtype)
    st = _lib.stream_of(dev)
    R = 3 if args.profile else 20
    ops = {}

    def record(name, fn, nbytes, note):
        _settle(torch, fn, ms=20.0)
        t = float(np.median(_events(torch, fn, R)))
        gbps = nbytes / (t * 1e-3) / 1e9
        ops[name] = {"ms": t, "algorithmic_bytes": int(nbytes), "GBps": gbps, "frac": gbps / PEAK["hbm_GBps"],
                     "bytes_counted": note}
        log(f"{name}: {t:.4f} ms, {nbytes / 1e6:.1f} MB -> {gbps:.0f} GB/s")

    # pooling k2 s2: the plan (cells -> order keys -> stable radix sort -> run heads -> scan), then the
    # value passes over its runs
    nb = ctypes.c_size_t()
    _lib.call("st_pool_workspace", N, ctypes.byref(nb))
    ws = torch.empty((max(nb.value, 1),), dtype=torch.uint8, device=dev)
    perm = torch.empty((N,), dtype=torch.int32, device=dev)
    seg = torch.empty((N + 1,), dtype=torch.int32, device=dev)
    inv = torch.empty((N,), dtype=torch.int32, device=dev)
    oc = torch.empty((N, 4), dtype=coords.dtype, device=dev)
    counts = torch.empty((2,), dtype=torch.int32, device=dev)

    def plan():
        _lib.call("st_pool_plan", _lib.ptr(coords), _lib.coord_code(coords.dtype), N, 2, 2, 0, _lib.ptr(ws),
                  nb.value, _lib.ptr(perm), _lib.ptr(seg), _lib.ptr(inv), _lib.ptr(oc), _lib.ptr(counts), st)

    plan()
    n_out = int(counts[0].item())
    # counted: its inputs and outputs only (coordinates read; perm, inverse, run starts and pooled
    # coordinates written) -- not the sort's own passes; left out of the aggregate value
    record("pool_plan_k2s2", plan, 8 * N + 12 * N + 8 * n_out,
           "coordinates read, perm / inverse / run starts / pooled coordinates written (the sort's passes not "
           "counted; not in the aggregate value)")
    out = torch.empty((n_out, C), dtype=dtype, device=dev)
    dout = torch.randn(n_out, C, generator=g).to(dev, dtype)
    dx = torch.empty((N, C), dtype=dtype, device=dev)
    for mode, mcode in (("max", 0), ("avg", 1)):
        record(f"pool_{mode}_forward", lambda: _lib.call(
            "st_pool_forward", _lib.ptr(X), C, fc, _lib.ptr(perm), _lib.ptr(seg), n_out, mcode, _lib.ptr(out), st),
            esz * (N + n_out) * C + 4 * (N + n_out), "features read once, pooled rows written, perm + run starts")
        extra = esz * (N + n_out) * C if mode == "max" else 0
        record(f"pool_{mode}_backward", lambda: _lib.call(
            "st_pool_backward", _lib.ptr(X), _lib.ptr(out), _lib.ptr(dout), N, C, fc, _lib.ptr(inv), _lib.ptr(seg),
            mcode, _lib.ptr(dx), st),
            esz * (n_out + N) * C + extra + 4 * (N + n_out),
            "pooled gradient read once, input gradient written" + (", inputs and outputs re-read (argmax)"
                                                                   if mode == "max" else "") + ", inverse + run starts")
    # upsampling x2: every row to its 8 children
    up = torch.empty((8 * N, C), dtype=dtype, device=dev)
    upc = torch.empty((8 * N, 4), dtype=coords.dtype, device=dev)
    record("upsample_x2_forward", lambda: _lib.call(
        "st_upsample", _lib.ptr(X), _lib.ptr(coords), _lib.coord_code(coords.dtype), N, C, fc, 2, _lib.ptr(up),
        _lib.ptr(upc), st), esz * 9 * N * C + 8 * 9 * N, "features read, 8 children written, coordinates alike")
    dup = torch.randn(8 * N, C, generator=g).to(dev, dtype)
    record("upsample_x2_backward", lambda: _lib.call(
        "st_upsample_backward", _lib.ptr(dup), N, C, fc, 2, _lib.ptr(dx), st),
        esz * 9 * N * C, "children's gradients read, summed rows written")
    # to_dense of the set max-pooled by 8 (a dense head's input: 4 x 180 x 180 x 5 cells)
    pooled = sparse_pooling(SparseTensor(X, coords, spatial_shape=shape, batch_size=4), 8, 0, 8, "max")
    pc, pf = pooled.C, pooled.F.contiguous()
    pshape = tuple(int(v) for v in pooled.spatial_shape)
    cells = 4 * pshape[0] * pshape[1] * pshape[2]
    grid = to_dense(pf, pc, pshape)
    B, sx, sy, sz = 4, *pshape
    # the C entry point (the Python wrapper first reads the batch count back to the host)
    record("to_dense_forward", lambda: _lib.call(
        "st_to_dense", _lib.ptr(pf), pf.shape[0], C, fc, _lib.ptr(pc), _lib.coord_code(pc.dtype), B, sx, sy, sz,
        _lib.ptr(grid), st),
        esz * cells * C + esz * pf.shape[0] * C + 8 * pf.shape[0],
        "the whole grid written (zeros included), rows and coordinates read")
    dgrid = torch.randn(tuple(grid.shape), generator=g).to(dev, dtype)
    dpf = torch.empty_like(pf)
    record("to_dense_backward", lambda: _lib.call(
        "st_from_dense", _lib.ptr(dgrid), B, sx, sy, sz, C, fc, _lib.ptr(pc), _lib.coord_code(pc.dtype),
        pf.shape[0], _lib.ptr(dpf), st),
        2 * esz * pf.shape[0] * C + 8 * pf.shape[0], "the rows' cells gathered, rows written, coordinates read")
    value_ops = [o for k, o in ops.items() if k != "pool_plan_k2s2"]
    tot_b = sum(o["algorithmic_bytes"] for o in value_ops)
    tot_t = sum(o["ms"] for o in value_ops)
    value = tot_b / (tot_t * 1e-3) / 1e9
    line = {
        "metric": "sparse pooling / upsampling / to_dense HBM GB/s (algorithmic bytes), 1 MI355X", "value": value,
        "unit": "GB/s", "n_gpus": 1, "steps": R, "warmup": 0, "clock_settle": {"ms": 20.0, "per_op": True},
        "ms_per_step": tot_t, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": args.dtype, "data": "synthetic (config-2 voxel set, N(0,1) features)",
        "config": {"workload": "spatial: max/avg pooling k2 s2, upsampling x2, to_dense of the set pooled by 8; "
                               "64 channels", "voxels": N, "pooled_k2": n_out, "pooled_k8": int(pf.shape[0]),
                   "dense_cells": cells, "channels": C},
        "ops": ops, "hbm_peak_GBps": PEAK["hbm_GBps"],
    }
    print(json.dumps(line))


def run_resnet(args):
    """SparseResNet21D (reference nn/backbones/resnet.py:81-109) forward + backward on the config-2
    voxel set with 4 input channels: 13 convolutions (4 strided), 13 per-sample batch norms with
    their ReLU / residual add fused, one JSON line.  A step takes a new SparseTensor over the same
    coordinates, so every kernel map, tile plan and pair list is rebuilt inside the step, as in a
    training loop over new scans; the step with the maps cached is logged beside it."""
    import torch

    from sparsetriton_amd import SparseTensor, workloads
    from sparsetriton_amd.config import set_fp32_precision
    from sparsetriton_amd.nn import SparseConv3DBase, SparseResNet21D

    set_fp32_precision(args.fp32_precision)
    dev = torch.device("cuda:0")
    dtype = {"f32": torch.float32, "bf16": torch.bfloat16}[args.dtype]
    seed = 0
    torch.manual_seed(seed)
    coords_np, shape = workloads.config2(seed=seed)
    coords = torch.as_tensor(coords_np, device=dev).to(torch.int16)
    N = coords.shape[0]
    g = torch.Generator(device="cpu").manual_seed(seed)
    X = torch.randn(N, 4, generator=g).to(dev, dtype)
    model = SparseResNet21D(in_channels=4).to(dev)
    convs = [m for m in model.modules() if isinstance(m, SparseConv3DBase)]
    for m in convs:
        m.to(dtype)  # batch-norm parameters and statistics stay fp32

    # useful flops: 2 P C_in C_out per pass; forward, input gradient (not for the first layer,
    # whose input is data) and weight gradient
    pairs = {}

    def hook(mod, inputs, output):
        t = inputs[0]
        k, s, d = mod.kernel_size[0], mod.stride[0], mod.dilation[0]
        p = ((k - 1) * d) // 2 if mod.subm else mod.padding[0]
        km = t._cache.neighbor_indices[(k, s, p, d, mod.subm, mod.transposed)][1]
        pairs[id(mod)] = km.num_pairs()

    hs = [m.register_forward_hook(hook) for m in convs]
    with torch.no_grad():
        outs = model(SparseTensor(X, coords, spatial_shape=shape, batch_size=4))
    for h in hs:
        h.remove()
    flops = sum(2.0 * pairs[id(m)] * m.in_channels * m.out_channels * (2 if i == 0 else 3)
                for i, m in enumerate(convs))
    grads = [torch.randn(tuple(o.F.shape), generator=g).to(dev, dtype) for o in outs]
    voxels = [int(o.F.shape[0]) for o in outs]
    del outs

    def step(sp):
        model.zero_grad(set_to_none=True)
        outs = model(sp)
        torch.autograd.backward([o.F for o in outs], grads)

    def timed(make, steps):
        _settle(torch, lambda: step(make()))
        for _ in range(args.warmup):
            step(make())
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step(make())
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    ms = timed(lambda: SparseTensor(X, coords, spatial_shape=shape, batch_size=4), args.steps)
    cached = SparseTensor(X, coords, spatial_shape=shape, batch_size=4)
    ms_cached = timed(lambda: cached, args.steps)

    # inference: evaluation mode under no_grad, where each block's batch norm, residual add and
    # ReLU run in its convolutions' GEMM stores (maps cached)
    model.eval()
    with torch.no_grad():
        _settle(torch, lambda: model(cached))
        for _ in range(args.warmup):
            model(cached)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            model(cached)
        e1.record()
        torch.cuda.synchronize()
    ms_infer = e0.elapsed_time(e1) / args.steps
    model.train()
    value = flops / (ms * 1e-3) / 1e12
    log(f"resnet21d {args.dtype}: N={N}, stage voxels {voxels}; step {ms:.3f} ms with map builds "
        f"({value:.2f} TFLOP/s), {ms_cached:.3f} ms with maps cached ({flops / (ms_cached * 1e-3) / 1e12:.2f}); "
        f"inference forward (eval, fused epilogues) {ms_infer:.3f} ms")
    line = {
        "metric": METRIC, "value": value, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "clock_settle": {"ms": SETTLE_MS}, "ms_per_step": ms, "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None, "dtype": args.dtype,
        "fp32_precision": args.fp32_precision if args.dtype == "f32" else None,
        "data": "synthetic (seeded LiDAR-like voxel set, N(0,1) features, random-init weights)",
        "config": {"workload": "resnet21d: SparseResNet21D(in_channels=4) fwd+bwd, config-2 voxel set, B=4, "
                               "maps rebuilt every step", "voxels": N, "stage_voxels": voxels,
                   "useful_flops_per_step": flops, "seed": seed},
        "ms_per_step_maps_cached": ms_cached,
        "inference_forward_ms_maps_cached": ms_infer,
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--dtype", choices=["f32", "bf16"], default="f32")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile", action="store_true",
                    help="short run for counter collection: few repetitions, plus a 256 MiB device copy whose "
                         "HBM counters calibrate the per-kernel traffic figures")
    ap.add_argument("--workload", choices=["config2", "resnet21d", "spatial"] + sorted(EXTRA), default="config2",
                    help="config2 is the headline; the others measure the other benchmark configurations")
    ap.add_argument("--fp32-precision", choices=["bf16x3", "ieee"], default="bf16x3",
                    help="fp32 matrix-core arithmetic (split-bf16 MFMA, the default, or IEEE fp32 MFMA)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the records of the other benchmark configurations in the default run")
    args = ap.parse_args()
    if args.workload != "config2":
        if args.gpus != 1:
            print("bench.py: one GPU only", file=sys.stderr)
            sys.exit(2)
        if args.workload == "spatial":
            return run_spatial(args)
        return run_resnet(args) if args.workload == "resnet21d" else run_extra(args)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); "
              "the sparse-convolution path is not sharded across GPUs here", file=sys.stderr)
        sys.exit(2)

    import torch

    from sparsetriton_amd import SparseTensor, workloads
    from sparsetriton_amd import _lib
    from sparsetriton_amd.nn.functional import sparse_conv3d
    from sparsetriton_amd.nn.functional.conv.conv import table_capacity
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import (
        gather_gemm_dgrad,
        gather_gemm_fwd,
        weight_prep,
        wgrad,
    )
    from sparsetriton_amd.nn.functional.conv.kmap import _target_offsets, subm_kernel_map
    from sparsetriton_amd.utils.hash import HashTable

    from sparsetriton_amd.config import set_fp32_precision

    set_fp32_precision(args.fp32_precision)
    dev = torch.device("cuda:0")
    dtype = {"f32": torch.float32, "bf16": torch.bfloat16}[args.dtype]
    Cin = Cout = 64
    seed = 0
    coords_np, shape = workloads.config2(seed=seed)
    N = coords_np.shape[0]
    rng = np.random.default_rng(seed)
    X_np = rng.standard_normal((N, Cin)).astype(np.float32)
    bound = 1.0 / np.sqrt(Cin * 27)
    W_np = rng.uniform(-bound, bound, (27, Cin, Cout)).astype(np.float32)
    dY_np = rng.standard_normal((N, Cout)).astype(np.float32)
    log(f"config2: N={N} voxels, shape={shape}, dtype={args.dtype}")

    coords = torch.as_tensor(coords_np, device=dev).to(torch.int16)
    offsets = _target_offsets(3, 1, 1, False, dev)

    # ------------------------------------------------ kernel-map build timing
    def build_kmap():
        # what sparse_conv3d does for a new coordinate set: the brick index and the neighbour query
        # in one launch, then the plans (mask-sorted tile plan; pair list and chunk order on a side
        # stream)
        km, _ = subm_kernel_map(coords, 4, shape, offsets, symmetric=True)
        km.prepare()
        return km

    for _ in range(3):
        build_kmap()
    torch.cuda.synchronize()
    kmap = build_kmap()
    kmap.symmetric  # resolves the duplicate / out-of-box check
    P = kmap.num_pairs()

    # the training step (forward + input and weight gradients through sparse_conv3d and autograd,
    # the map cached on the tensor)
    X = torch.as_tensor(X_np, device=dev).to(dtype)
    dY = torch.as_tensor(dY_np, device=dev).to(dtype)
    w = torch.as_tensor(W_np, device=dev).to(dtype).requires_grad_(True)
    feats = X.clone().requires_grad_(True)
    sp = SparseTensor(feats, coords, spatial_shape=shape, batch_size=4)
    sp._cache.neighbor_indices[(3, 1, 1, 1, True, False)] = (sp.C, kmap, sp.spatial_shape)

    def step():
        feats.grad = None
        w.grad = None
        out = sparse_conv3d(sp, w, 3)
        out.F.backward(dY)

    settled = {"ms": SETTLE_MS, "steps_before_map_timing": _settle(torch, step)}
    R = 3 if args.profile else 20
    kmap_t = _events(torch, build_kmap, R)
    log(f"pairs P={P} (P/N={P / N:.2f}); kmap build median {np.median(kmap_t):.3f} ms")

    # per-stage kernel timings of the map build
    table = HashTable(table_capacity(N), device=dev)

    def t_insert():  # the hash table itself (strided / transposed / hash-fly paths use it)
        table.clear()
        table.insert(coords)
        table.table_keys  # runs the deferred clear + insert

    ins_t = _events(torch, t_insert, R)
    table.check()
    q_t = _events(torch, lambda: subm_kernel_map(coords, 4, shape, offsets, symmetric=False), R)
    prep_t = _events(torch, lambda: subm_kernel_map(coords, 4, shape, offsets, symmetric=True)[0].prepare(),
                     R) - np.median(q_t)

    # --------------------------------------------------------- train step
    settled["steps_before_step_timing"] = _settle(torch, step)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t_wall) * 1e3
    ms_per_step = e0.elapsed_time(e1) / args.steps
    flops_step = 6.0 * P * Cin * Cout
    value = flops_step / (ms_per_step * 1e-3) / 1e12
    log(f"step {ms_per_step:.3f} ms (wall {wall_ms / args.steps:.3f} ms) -> {value:.2f} TFLOP/s")

    # ---------------------------------------------- per-kernel (events) timing
    wt = weight_prep(w.detach(), _lib.W_TRANSPOSE)
    wd = w.detach().contiguous()
    KR = 5 if args.profile else 30
    kern = {"gather_gemm_fwd": _events_batch(torch, lambda: gather_gemm_fwd(X, kmap, wt), KR),
            "gather_gemm_dgrad": _events_batch(torch, lambda: gather_gemm_dgrad(dY, kmap, wd), KR),
            "wgrad(+reduce)": _events_batch(torch, lambda: wgrad(X, dY, kmap, w.dtype), KR)}
    dom = max(kern, key=kern.get)
    dkey = args.dtype if args.dtype != "f32" else f"f32-{args.fp32_precision}"
    traffic, traffic_src = _measured_traffic(dkey, dom)
    roofline = gemm_roofline(dom, kern[dom], N, N, Cin, Cout, 27, P, args.dtype, args.fp32_precision,
                             traffic=traffic, traffic_source=traffic_src)
    tflops = roofline["mfma_TFLOPs"]
    T = table.capacity
    ins_bytes = 8 * N + 12 * T + 12 * N  # int16 coords read + table clear + one slot written per insert
    # submanifold map (brick index + query, one launch), by the fixed formula 16 N + 12 Q + 4 N K:
    # coordinates read, one 12-byte slot-equivalent read per in-bound query, the (K, N) map written
    off_np = offsets.cpu().numpy()
    Q = int(sum(((coords_np[:, 1:] - o >= 0) & (coords_np[:, 1:] - o < np.array(shape))).all(axis=1).sum()
                for o in off_np))
    q_bytes = 16 * N + 12 * Q + 4 * 27 * N
    kmap_info = {
        "kmap_build_ms": _stats(kmap_t),
        "hash_insert_ms": float(np.median(ins_t)), "hash_insert_GBps": ins_bytes / (np.median(ins_t) * 1e-3) / 1e9,
        "subm_index_and_query_ms": float(np.median(q_t)),
        "subm_index_and_query_GBps": q_bytes / (np.median(q_t) * 1e-3) / 1e9,
        "in_bound_queries": Q,
        "plans_ms": float(np.median(prep_t)),
    }
    log(f"kernels (avg ms): {kern}; roofline {dom}: {roofline['achieved']:.1f} {roofline['unit']} = "
        f"{roofline['frac'] * 100:.1f}% of the {roofline['bound']} peak; MFMA {tflops:.1f} TFLOP/s")

    if args.profile:
        # calibration for HBM counters: a plain device copy of 256 MiB (reads and writes 262144 KiB)
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # the other BASELINE configurations, each a record with its own step time, effective rate,
    # dominant kernel and roofline (the headline's voxel set is reused)
    configs = None
    if not args.no_configs and not args.profile:
        configs = {}
        cache = {"config2": (coords_np, shape)}
        for name in DEFAULT_CONFIGS:
            configs[name] = measure_extra(name, min(args.steps, 20), min(args.warmup, 5), False,
                                          args.fp32_precision, coords_cache=cache)
        set_fp32_precision(args.fp32_precision)
        torch.cuda.empty_cache()

    cfg1_gpu = gpu_config1(torch, 5 if args.profile else 50)
    log(f"config 1 on the GPU: step {cfg1_gpu['fwd_bwd_step_ms']['median']:.3f} ms, "
        f"first call {cfg1_gpu['first_call_build_plus_fwd_ms']['median']:.3f} ms")
    cpu = None
    if not args.no_cpu:
        W_use = torch.as_tensor(W_np).to(dtype).float().numpy()
        X_use = X.float().cpu().numpy()
        dY_use = dY.float().cpu().numpy()
        cpu = cpu_baseline(coords_np, shape, X_use, W_use, dY_use, profile=args.profile)
        c1 = cpu["config1"]
        log(f"cpu baseline: config 2 {cpu['value'] * 1e3:.2f} GFLOP/s on {cpu['cores']} threads; config 1 "
            f"{c1['all']['fwd_bwd_GFLOPs']['median']:.2f} GFLOP/s ({c1['all']['threads']} threads), "
            f"{c1['one']['fwd_bwd_GFLOPs']['median']:.2f} GFLOP/s (1 thread)")

    peaks = None
    if not args.profile:
        peaks = measured_peaks(torch, dev)
        log(f"measured peaks: copy {peaks['hbm_copy_GBps']:.0f} GB/s, bf16 MFMA {peaks['bf16_mfma_TFLOPs']:.0f} "
            f"TFLOP/s (spec {PEAK['hbm_GBps']:.0f} GB/s, {PEAK['bf16_TFLOPs']:.0f} TFLOP/s)")
        with_measured_peak(roofline, peaks)
        for rec in (configs or {}).values():
            with_measured_peak(rec.get("roofline"), peaks)

    line = {
        "metric": METRIC,
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_settle": settled,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "fp32_precision": args.fp32_precision if args.dtype == "f32" else None,
        "data": "synthetic (seeded LiDAR-like voxel set, N(0,1) features)",
        "config": {"workload": "config2: SubMConv3D 64->64 k3, B=4, 1440x1440x41 LiDAR-like grid",
                   "voxels": N, "pairs": P, "pairs_per_voxel": P / N, "C_in": Cin, "C_out": Cout, "seed": seed},
        "kmap_build_ms": float(np.median(kmap_t)),
        "kmap": kmap_info,
        "kernels_avg_ms": kern,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "gpu_config1": cfg1_gpu,
        "configs": configs,
        "measured_peaks": peaks,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
