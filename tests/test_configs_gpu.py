"""BASELINE configurations 1 to 5 on the GPU, every output and gradient tensor at full size
against the float64 oracle.

Inputs are quantised to the compute dtype first, so the oracle sees the operands the kernels see.
Tolerances (relative Frobenius error per tensor): fp32 2e-3, bf16 2e-2 -- the north-star bounds.
Output coordinates and kernel maps are compared bit for bit.  The adjoint identities
<dY, Y> = <dX, X> = <dW, W> are checked beside the per-tensor comparison.

  config 1  SubMConv3D 16->32 k3, B=2, 64^3, 4096 uniform voxels, fp32 and bf16, both algorithms
  config 2  SubMConv3D 64->64 k3, B=4, 1440x1440x41 LiDAR-like set (the benchmark's headline
            workload), fp32 and bf16, both algorithms: ImplicitHashFlyGEMM runs the brick-index
            lookups inside the GEMM at 64 channels, its forward and weight gradient bitwise equal
            to PrecomputedNeighborGEMM's
  config 3  SparseConv3D 64->128 k3 s2 p1 fp32 on the config-2 set, both algorithms
  config 4  SparseConvTransposed3D 128->64 k3 s2 p1 bf16 on config 3's output coordinates
  config 5  SubMConv3D 128->128 k3 bf16, 1M voxels of 2-voxel walls in 256^3, PrecomputedNeighborGEMM
            vs ImplicitHashFlyGEMM (reference implicit_hashfly_gemm.py:45-148 vs
            implicit_precomputed_gemm.py:64-126)
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from sparsetriton_amd import SparseTensor, workloads
from sparsetriton_amd.config import ConvAlgo, set_conv_algo
from sparsetriton_amd.nn.functional import sparse_conv3d

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 2e-3, torch.bfloat16: 2e-2}


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _q(a: np.ndarray, dtype) -> np.ndarray:
    return torch.as_tensor(np.ascontiguousarray(a, dtype=np.float32)).to(dtype).float().numpy()


def _inputs(seed, n_in, n_out, cin, cout, dtype):
    rng = np.random.default_rng(seed)
    X = _q(rng.standard_normal((n_in, cin)), dtype)
    bound = 1.0 / np.sqrt(cin * 27)  # the modules' U(+-1/sqrt(C_in K)) init
    W = _q(rng.uniform(-bound, bound, (27, cin, cout)), dtype)
    dY = _q(rng.standard_normal((n_out, cout)), dtype)
    return X, W, dY


def _gpu(device, c, shape, batch, X, W, dY, dtype, algo, **conv):
    set_conv_algo(algo)
    feats = torch.as_tensor(X, device=device).to(dtype).requires_grad_(True)
    w = torch.as_tensor(W, device=device).to(dtype).requires_grad_(True)
    sp = SparseTensor(feats, torch.as_tensor(c, device=device).to(torch.int16), spatial_shape=shape, batch_size=batch)
    out = sparse_conv3d(sp, w, 3, **conv)
    if dY is not None:
        out.F.backward(torch.as_tensor(dY, device=device).to(dtype))
    return sp, out, feats.grad, w.grad


def _adjoint(X, W, dY, y, dX, dW, tol):
    """<dY, Y> = <dX, X> = <dW, W>: the convolution is linear in X and in W."""
    s_y = float(np.vdot(dY, y))
    s_x = float(np.vdot(dX, X))
    s_w = float(np.vdot(dW, W))
    assert abs(s_x - s_y) <= tol * abs(s_y) and abs(s_w - s_y) <= tol * abs(s_y), (s_y, s_x, s_w)


def _compare(out, dX, dW, ref, tol, what):
    y, gx, gw = ref
    errs = (rel(out.F.detach().float().cpu(), y), rel(dX.float().cpu(), gx), rel(dW.float().cpu(), gw))
    print(f"{what}: rel err fwd {errs[0]:.2e} dX {errs[1]:.2e} dW {errs[2]:.2e}", flush=True)
    assert max(errs) < tol, (what, errs)
    return errs


# ------------------------------------------------------------------- config 1

@pytest.mark.parametrize("algo", list(ConvAlgo))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config1_subm16x32(device, dtype, algo):
    c, shape = workloads.config1(seed=0)
    n = c.shape[0]
    X, W, dY = _inputs(1, n, n, 16, 32, dtype)
    sp, out, dX, dW = _gpu(device, c, shape, 2, X, W, dY, dtype, algo)
    assert torch.equal(out.C, sp.C)
    nbr = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, shape)
    ref = (O.fwd_f64(X, W, nbr), O.dgrad_f64(dY, W, nbr, n), O.wgrad_f64(X, dY, nbr, 27))
    _compare(out, dX, dW, ref, TOL[dtype], f"config1 {dtype} {algo.value}")
    assert (nbr >= 0).sum() > n  # the centre offset alone gives n pairs
    if algo == ConvAlgo.PrecomputedNeighborGEMM:
        kmap = sp._cache.neighbor_indices[(3, 1, 1, 1, True, False)][1]
        assert (kmap.neighbor_indices.cpu().numpy() == nbr).all()


# ------------------------------------------------------------------- config 2

@pytest.fixture(scope="module")
def cfg2_map():
    c, shape = workloads.config2(seed=0)
    nbr = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, shape)
    return c, shape, nbr


_CFG2 = {}


def _cfg2_case(cfg2_map, dtype):
    """Inputs and float64 references of config 2 in `dtype` (built once per dtype)."""
    if dtype not in _CFG2:
        c, shape, nbr = cfg2_map
        n = c.shape[0]
        X, W, dY = _inputs(2, n, n, 64, 64, dtype)
        ref = (O.fwd_f64_blas(X, W, nbr), O.dgrad_f64_blas(dY, W, nbr, n), O.wgrad_f64_blas(X, dY, nbr, 27))
        _CFG2[dtype] = (X, W, dY, ref, {})
    return _CFG2[dtype]


@pytest.mark.parametrize("algo", list(ConvAlgo))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config2_subm64x64(device, cfg2_map, dtype, algo):
    c, shape, nbr = cfg2_map
    X, W, dY, ref, done = _cfg2_case(cfg2_map, dtype)
    sp, out, dX, dW = _gpu(device, c, shape, 4, X, W, dY, dtype, algo)
    assert c.shape[0] == 470_532 and torch.equal(out.C, sp.C)
    _compare(out, dX, dW, ref, TOL[dtype], f"config2 {dtype} {algo.value}")
    _adjoint(X, W, dY, out.F.detach().double().cpu().numpy(), dX.double().cpu().numpy(),
             dW.double().cpu().numpy(), TOL[dtype])
    if algo == ConvAlgo.PrecomputedNeighborGEMM:
        kmap = sp._cache.neighbor_indices[(3, 1, 1, 1, True, False)][1]
        assert (kmap.neighbor_indices.cpu().numpy() == nbr).all()
        assert kmap.symmetric
    else:
        from sparsetriton_amd.nn.functional.conv.kmap import BrickIndex

        # the brick-index lookups inside the GEMM ran (no kernel map was stored)
        assert isinstance(sp._cache.kmaps.get(("brick_index", 4, tuple(shape))), BrickIndex)
        assert not sp._cache.neighbor_indices
    done[algo] = (out.F.detach().clone(), dX.clone(), dW.clone())
    if len(done) == 2:
        # forward and weight gradient bitwise equal across the algorithms (same per-row offset
        # order, same pair list); the input gradients agree to rounding
        pre, fly = done[ConvAlgo.PrecomputedNeighborGEMM], done[ConvAlgo.ImplicitHashFlyGEMM]
        assert torch.equal(pre[0], fly[0]) and torch.equal(pre[2], fly[2])
        assert rel(pre[1].float().cpu(), fly[1].float().cpu()) < TOL[dtype] / 4
        del _CFG2[dtype]


# ------------------------------------------------------------- configs 3, 4

@pytest.fixture(scope="module")
def cfg3():
    """Config-2 voxels, the strided geometry's output coordinates and exact map (oracle)."""
    c, shape = workloads.config2(seed=0)
    off = O.target_offsets(3, 1, 1, False)
    ns = O.out_shape(shape, 3, 2, 1, 1, False)
    oc = O.out_coords(c, off, 2, False, ns)
    nbr = O.exact_kmap(c, oc, off, 2, shape)
    return c, shape, oc, ns, nbr


@pytest.fixture(scope="module")
def cfg3_ref(cfg3):
    c, shape, oc, ns, nbr = cfg3
    X, W, dY = _inputs(3, c.shape[0], oc.shape[0], 64, 128, torch.float32)
    ref = (O.fwd_f64_blas(X, W, nbr), O.dgrad_f64_blas(dY, W, nbr, c.shape[0]), O.wgrad_f64_blas(X, dY, nbr, 27))
    return X, W, dY, ref


@pytest.mark.parametrize("algo", list(ConvAlgo))
def test_config3_strided64x128_f32(device, cfg3, cfg3_ref, algo):
    c, shape, oc, ns, nbr = cfg3
    X, W, dY, ref = cfg3_ref
    sp, out, dX, dW = _gpu(device, c, shape, 4, X, W, dY, torch.float32, algo, stride=2, padding=1,
                           submanifold=False)
    assert tuple(out.spatial_shape) == tuple(ns) == (720, 720, 21)
    assert (out.C.int().cpu().numpy() == oc).all()  # same coordinates in the same order
    _compare(out, dX, dW, ref, TOL[torch.float32], f"config3 {algo.value}")
    _adjoint(X, W, dY, out.F.detach().double().cpu().numpy(), dX.double().cpu().numpy(),
             dW.double().cpu().numpy(), TOL[torch.float32])


@pytest.fixture(scope="module")
def cfg4(cfg3):
    """Config 3's output coordinates as input, the transposed geometry's outputs and exact map."""
    _, _, c3, ns3, _ = cfg3
    off = O.target_offsets(3, 1, 1, True)
    ns = O.out_shape(ns3, 3, 2, 1, 1, True)
    oc = O.out_coords(c3, off, 2, True, ns)
    nbr = O.exact_kmap(c3, oc, off, 1, tuple(v * 2 for v in ns3), in_scale=2)
    return c3, ns3, oc, ns, nbr


@pytest.fixture(scope="module")
def cfg4_ref(cfg4):
    c, shape, oc, ns, nbr = cfg4
    X, W, dY = _inputs(4, c.shape[0], oc.shape[0], 128, 64, torch.bfloat16)
    return X, W, dY, (O.fwd_f64_blas(X, W, nbr), O.dgrad_f64_blas(dY, W, nbr, c.shape[0]),
                      O.wgrad_f64_blas(X, dY, nbr, 27))


def test_config4_transposed128x64_bf16(device, cfg4, cfg4_ref):
    c, shape, oc, ns, nbr = cfg4
    X, W, dY, ref = cfg4_ref
    sp, out, dX, dW = _gpu(device, c, shape, 4, X, W, dY, torch.bfloat16, ConvAlgo.PrecomputedNeighborGEMM,
                           stride=2, padding=1, transposed=True, submanifold=False)
    assert tuple(out.spatial_shape) == tuple(ns) == (1439, 1439, 41)
    assert (out.C.int().cpu().numpy() == oc).all()
    kmap = sp._cache.neighbor_indices[(3, 2, 1, 1, False, True)][1]
    assert (kmap.neighbor_indices.cpu().numpy() == nbr).all()
    _compare(out, dX, dW, ref, TOL[torch.bfloat16], "config4 precomputed")
    _adjoint(X, W, dY, out.F.detach().double().cpu().numpy(), dX.double().cpu().numpy(),
             dW.double().cpu().numpy(), TOL[torch.bfloat16])


def test_config4_transposed_hashfly_bf16(device, cfg4, cfg4_ref):
    c, shape, oc, ns, nbr = cfg4
    X, W, dY, ref = cfg4_ref
    sp, out, dX, dW = _gpu(device, c, shape, 4, X, W, dY, torch.bfloat16, ConvAlgo.ImplicitHashFlyGEMM,
                           stride=2, padding=1, transposed=True, submanifold=False)
    assert (out.C.int().cpu().numpy() == oc).all()
    _compare(out, dX, dW, ref, TOL[torch.bfloat16], "config4 hashfly")


# ------------------------------------------------------------------- config 5

@pytest.fixture(scope="module")
def cfg5():
    c, shape = workloads.config5(seed=0)
    nbr = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, shape)
    X, W, dY = _inputs(5, c.shape[0], c.shape[0], 128, 128, torch.bfloat16)
    ref = (O.fwd_f64_blas(X, W, nbr), O.dgrad_f64_blas(dY, W, nbr, c.shape[0]), O.wgrad_f64_blas(X, dY, nbr, 27))
    return c, shape, nbr, X, W, dY, ref


@pytest.fixture(scope="module")
def cfg5_precomputed(device, cfg5):
    c, shape, nbr, X, W, dY, ref = cfg5
    sp, out, dX, dW = _gpu(device, c, shape, 1, X, W, dY, torch.bfloat16, ConvAlgo.PrecomputedNeighborGEMM)
    kmap = sp._cache.neighbor_indices[(3, 1, 1, 1, True, False)][1]
    return sp, kmap, out.F.detach().clone(), dX.clone(), dW.clone()


def test_config5_map_exact(device, cfg5, cfg5_precomputed):
    c, shape, nbr = cfg5[:3]
    _, kmap, _, _, _ = cfg5_precomputed
    assert c.shape[0] == 1_000_000
    assert (kmap.neighbor_indices.cpu().numpy() == nbr).all()
    assert kmap.symmetric  # unique in-box coordinates: the input gradient reads the map backwards


def test_config5_subm128_precomputed_bf16(device, cfg5, cfg5_precomputed):
    c, shape, nbr, X, W, dY, ref = cfg5
    sp, kmap, y, dX, dW = cfg5_precomputed
    errs = (rel(y.float().cpu(), ref[0]), rel(dX.float().cpu(), ref[1]), rel(dW.float().cpu(), ref[2]))
    print(f"config5 precomputed: rel err {errs}", flush=True)
    assert max(errs) < TOL[torch.bfloat16], errs
    _adjoint(X, W, dY, y.double().cpu().numpy(), dX.double().cpu().numpy(), dW.double().cpu().numpy(),
             TOL[torch.bfloat16])


def test_config5_hashfly_vs_precomputed_bf16(device, cfg5, cfg5_precomputed):
    c, shape, nbr, X, W, dY, ref = cfg5
    _, _, y_pre, dX_pre, dW_pre = cfg5_precomputed
    sp, out, dX, dW = _gpu(device, c, shape, 1, X, W, dY, torch.bfloat16, ConvAlgo.ImplicitHashFlyGEMM)
    # both algorithms accumulate each output row's offsets in the same order: the forward agrees bitwise
    assert torch.equal(out.F, y_pre)
    _compare(out, dX, dW, ref, TOL[torch.bfloat16], "config5 hashfly")
    # the gradients sum in different fixed orders: equal to within bf16 rounding
    assert rel(dX.float().cpu(), dX_pre.float().cpu()) < 1e-2
    assert rel(dW.float().cpu(), dW_pre.float().cpu()) < 1e-2
