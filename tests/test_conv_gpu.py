"""Sparse convolution forward / input gradient / weight gradient on the GPU.

Tolerances (relative Frobenius error vs float64, per output tensor):
fp32 2e-3, bf16 2e-2, fp16 1e-2 -- the north-star bounds.  fp32 runs in the
default split-bf16 mode (three bf16 MFMAs per product) unless a test selects
IEEE fp32; both land far inside, and test_fp32_precision_modes pins each
mode's own accuracy.  The reference's own test tolerances
(atol = rtol = 1e-3 forward, 5e-2 gradients, fp16; tests/test_sparse_conv.py)
are applied on its parametrisations against dense convolution.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O
from sparsetriton_amd import SparseTensor, randn, workloads
from sparsetriton_amd.config import ConvAlgo, set_conv_algo
from sparsetriton_amd.nn import SparseConv3D, SparseConvTransposed3D, SubMConv3D
from sparsetriton_amd.nn.functional import sparse_conv3d

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
TOL = {torch.float32: 2e-3, torch.bfloat16: 2e-2, torch.float16: 1e-2}


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _rand_coords(rng, n, S, B=2):
    lin = np.sort(rng.choice(B * S ** 3, n, replace=False))
    return np.stack([lin // S ** 3, (lin // S ** 2) % S, (lin // S) % S, lin % S], 1).astype(np.int32)


def _run(device, c, shape, X, W, dY, k, s, p, d, tr, subm, dtype, algo):
    set_conv_algo(algo)
    feats = torch.as_tensor(X, device=device).to(dtype).requires_grad_(True)
    w = torch.as_tensor(W, device=device).to(dtype).requires_grad_(True)
    sp = SparseTensor(feats, torch.as_tensor(c, device=device), spatial_shape=shape)
    out = sparse_conv3d(sp, w, k, stride=s, padding=p, dilation=d, transposed=tr, submanifold=subm)
    out.F.backward(torch.as_tensor(dY, device=device).to(dtype))
    return out, feats.grad, w.grad


def _oracle(c, oc, shape, X, W, dY, k, s, p, d, tr):
    off = O.target_offsets(k, d, p, tr)
    if tr:
        nbr = O.exact_kmap(c, oc, off, 1, tuple(v * s for v in shape), in_scale=s)
    else:
        nbr = O.exact_kmap(c, oc, off, s, shape)
    return O.fwd_f64(X, W, nbr), O.dgrad_f64(dY, W, nbr, c.shape[0]), O.wgrad_f64(X, dY, nbr, k ** 3)


# ------------------------------------------------------------- golden cases

def _golden():
    z = np.load(GOLD / "conv_cases.npz")
    return z, sorted({k.split("/")[0] for k in z.files})


@pytest.mark.parametrize("algo", list(ConvAlgo))
@pytest.mark.parametrize("name", _golden()[1])
def test_golden_dense_cases(device, name, algo):
    z, _ = _golden()
    g = lambda key: z[f"{name}/{key}"]
    C_in, C_out, k, s, p, d, tr, subm = (int(v) for v in g("meta"))
    c, X, W = g("coords"), g("feats"), g("weight")
    shape = tuple(int(v) for v in g("spatial_shape"))
    gold_rows = {tuple(r): i for i, r in enumerate(g("out_coords").tolist())}
    # the GPU output order is its own (first occurrence); dY is given per golden row
    set_conv_algo(algo)
    feats = torch.as_tensor(X, device=device).requires_grad_(True)
    w = torch.as_tensor(W, device=device).requires_grad_(True)
    sp = SparseTensor(feats, torch.as_tensor(c, device=device), spatial_shape=shape)
    out = sparse_conv3d(sp, w, k, stride=s, padding=p, dilation=d, transposed=bool(tr), submanifold=bool(subm))
    oc = out.C.cpu().numpy()
    assert oc.shape[0] == len(gold_rows)
    perm = np.array([gold_rows[tuple(r)] for r in oc.tolist()])
    assert rel(out.F.detach().cpu(), g("out")[perm]) < 1e-5
    out.F.backward(torch.as_tensor(g("dY")[perm], device=device))
    assert rel(feats.grad.cpu(), g("dX")) < 1e-5
    assert rel(w.grad.cpu(), g("dW")) < 1e-5
    if subm:
        assert out.C is sp.C and out._cache is sp._cache


# --------------------------------------------------- dtype / channel matrix

CHANNELS = [(4, 8), (16, 32), (64, 64), (64, 128), (128, 64), (3, 5), (20, 36), (128, 128), (256, 32)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cin,cout", CHANNELS)
def test_subm_dtypes_channels(device, dtype, cin, cout):
    rng = np.random.default_rng(cin * 1000 + cout)
    c = _rand_coords(rng, 4000, 20)
    X = rng.standard_normal((4000, cin)).astype(np.float32)
    W = (rng.standard_normal((27, cin, cout)) / np.sqrt(27 * cin)).astype(np.float32)
    dY = rng.standard_normal((4000, cout)).astype(np.float32)
    # quantise inputs to the compute dtype so the oracle sees the same operands
    Xq = torch.as_tensor(X).to(dtype).float().numpy()
    Wq = torch.as_tensor(W).to(dtype).float().numpy()
    dYq = torch.as_tensor(dY).to(dtype).float().numpy()
    out, dX, dW = _run(device, c, (20, 20, 20), Xq, Wq, dYq, 3, 1, 1, 1, False, True, dtype,
                       ConvAlgo.PrecomputedNeighborGEMM)
    y, gx, gw = _oracle(c, c, (20, 20, 20), Xq, Wq, dYq, 3, 1, 1, 1, False)
    tol = TOL[dtype]
    assert out.F.dtype == dtype and dX.dtype == dtype and dW.dtype == dtype
    assert rel(out.F.detach().float().cpu(), y) < tol
    assert rel(dX.float().cpu(), gx) < tol
    assert rel(dW.float().cpu(), gw) < tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("k,s,p,d,tr", [(3, 2, 1, 1, False), (3, 2, 1, 1, True), (5, 1, 2, 1, False),
                                        (3, 1, 1, 1, True), (3, 2, 1, 2, False)])
def test_general_geometries(device, dtype, k, s, p, d, tr):
    rng = np.random.default_rng(k + 10 * s + 100 * p + tr)
    shape = (16, 16, 16)
    c = _rand_coords(rng, 2500, 16)
    X = torch.as_tensor(rng.standard_normal((2500, 32)).astype(np.float32)).to(dtype).float().numpy()
    W = torch.as_tensor((rng.standard_normal((k ** 3, 32, 48)) / np.sqrt(32 * k ** 3)).astype(np.float32)).to(
        dtype).float().numpy()
    for algo in ConvAlgo:
        set_conv_algo(algo)
        feats = torch.as_tensor(X, device=device).to(dtype).requires_grad_(True)
        w = torch.as_tensor(W, device=device).to(dtype).requires_grad_(True)
        sp = SparseTensor(feats, torch.as_tensor(c, device=device), spatial_shape=shape)
        out = sparse_conv3d(sp, w, k, stride=s, padding=p, dilation=d, transposed=tr, submanifold=False)
        oc = out.C.cpu().numpy()
        dY = torch.as_tensor(rng.standard_normal((oc.shape[0], 48)).astype(np.float32)).to(dtype).float().numpy()
        out.F.backward(torch.as_tensor(dY, device=device).to(dtype))
        y, gx, gw = _oracle(c, oc, shape, X, W, dY, k, s, p, d, tr)
        tol = TOL[dtype]
        assert rel(out.F.detach().float().cpu(), y) < tol, algo
        assert rel(feats.grad.float().cpu(), gx) < tol, algo
        assert rel(w.grad.float().cpu(), gw) < tol, algo


@pytest.mark.parametrize("algo", list(ConvAlgo))
@pytest.mark.parametrize("case", ["in_box", "out_of_box", "duplicates", "both", "repeats_outside"])
def test_subm_rows_outside_shape_or_repeated(device, algo, case):
    """Submanifold fwd + dX + dW when rows lie outside spatial_shape or repeat a coordinate.

    Such a map is not its own transpose: a row outside the shape keeps its in-bounds
    neighbours (the reference bounds the neighbour only, conv.py:55-59) but no row finds it,
    and a repeated coordinate resolves to its lowest row.  The input gradient must still be
    the adjoint of the forward -- the reference's scatter over the forward map
    (implicit_precomputed_gemm.py:129-177), which the oracle's dgrad restates."""
    rng = np.random.default_rng(31)
    n, S = 2000, 20
    c = _rand_coords(rng, n, S)
    shape = (S, S, S)
    if case in ("out_of_box", "both"):
        shape = (15, 18, 20)
    if case in ("duplicates", "both"):
        rows = rng.choice(n, 150, replace=False)
        c[rows[75:]] = c[rows[:75]]  # 75 rows repeat another row's coordinate
    if case == "repeats_outside":
        # repeats only among rows just past the box (z = 15): the brick index does not hold those
        # rows, so its duplicate count cannot see them, yet two such rows reach the same
        # (input, offset) -- the transposed map must fold them, as for repeats inside the box
        shape = (20, 20, 15)
        outside = np.flatnonzero(c[:, 3] == 15)
        rows = rng.choice(outside, 40, replace=False)
        c[rows[20:]] = c[rows[:20]]
        nbr = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, shape)
        assert any(len(v[v >= 0]) > len(np.unique(v[v >= 0])) for v in nbr.T)  # the case is exercised
    X = rng.standard_normal((n, 32)).astype(np.float32)
    W = (rng.standard_normal((27, 32, 24)) / np.sqrt(27 * 32)).astype(np.float32)
    dY = rng.standard_normal((n, 24)).astype(np.float32)
    set_conv_algo(algo)
    feats = torch.as_tensor(X, device=device).requires_grad_(True)
    w = torch.as_tensor(W, device=device).requires_grad_(True)
    sp = SparseTensor(feats, torch.as_tensor(c, device=device), spatial_shape=shape, batch_size=2)
    out = sparse_conv3d(sp, w, 3)
    out.F.backward(torch.as_tensor(dY, device=device))
    y, gx, gw = _oracle(c, c, shape, X, W, dY, 3, 1, 1, 1, False)
    assert rel(out.F.detach().cpu(), y) < 1e-4
    assert rel(feats.grad.cpu(), gx) < 1e-4, case
    assert rel(w.grad.cpu(), gw) < 1e-4
    if algo == ConvAlgo.PrecomputedNeighborGEMM:
        kmap = sp._cache.neighbor_indices[(3, 1, 1, 1, True, False)][1]
        assert kmap.symmetric == (case == "in_box")
    else:
        gl = sp._cache.kmaps[("hashfly", 3, 1, 1, 1, True, False)][3]
        assert gl.usable() == (case in ("in_box", "out_of_box"))


@pytest.mark.parametrize("algo", list(ConvAlgo))
def test_unpackable_coordinates_raise(device, algo):
    """A coordinate the table cannot key (negative batch) raises instead of silently losing its
    row's neighbours."""
    c = _rand_coords(np.random.default_rng(32), 500, 12)
    c[7, 0] = -1
    set_conv_algo(algo)
    sp = SparseTensor(torch.randn(500, 8, device=device), torch.as_tensor(c, device=device),
                      spatial_shape=(12, 12, 12), batch_size=2)
    with pytest.raises(RuntimeError, match="packable range"):
        sparse_conv3d(sp, torch.randn(27, 8, 8, device=device), 3)


def test_mixed_precision_weight_grad_dtype(device):
    # bf16 activations with fp32 master weights: dW comes back in fp32
    rng = np.random.default_rng(2)
    c = _rand_coords(rng, 1000, 12)
    feats = torch.randn(1000, 16, device=device, dtype=torch.bfloat16, requires_grad=True)
    conv = SubMConv3D(16, 16, 3).to(device)
    out = conv(SparseTensor(feats, torch.as_tensor(c, device=device), spatial_shape=(12, 12, 12)))
    out.F.float().sum().backward()
    assert out.F.dtype == torch.bfloat16 and conv.weight.grad.dtype == torch.float32
    assert feats.grad.dtype == torch.bfloat16 and conv.bias.grad is not None


# ---------------------------------------------- algorithms / determinism

@pytest.mark.parametrize("algo", list(ConvAlgo))
@pytest.mark.parametrize("precision,bound", [("bf16x3", 1e-4), ("ieee", 2e-5)])
@pytest.mark.parametrize("cin,cout", [(64, 64), (32, 48), (64, 128)])
def test_fp32_precision_modes(device, algo, precision, bound, cin, cout):
    # Split-bf16 products carry <= ~2^-15 relative error (TF32: 2^-11); the sums
    # of a few hundred products land near 1e-5 relative.  IEEE fp32 lands near 1e-6.
    from sparsetriton_amd.config import set_fp32_precision
    set_fp32_precision(precision)
    rng = np.random.default_rng(cin + cout)
    c = _rand_coords(rng, 5000, 20)
    X = rng.standard_normal((5000, cin)).astype(np.float32)
    W = (rng.standard_normal((27, cin, cout)) / np.sqrt(27 * cin)).astype(np.float32)
    dY = rng.standard_normal((5000, cout)).astype(np.float32)
    out, gx, gw = _run(device, c, (20, 20, 20), X, W, dY, 3, 1, 1, 1, False, True, torch.float32, algo)
    f, dx, dw = _oracle(c, c, (20, 20, 20), X, W, dY, 3, 1, 1, 1, False)
    errs = (rel(out.F.detach().cpu(), f), rel(gx.cpu(), dx), rel(gw.cpu(), dw))
    assert max(errs) < bound, errs
    if precision == "bf16x3":  # the split kernels really ran: IEEE fp32 rounds differently
        set_fp32_precision("ieee")
        out2, _, _ = _run(device, c, (20, 20, 20), X, W, dY, 3, 1, 1, 1, False, True, torch.float32, algo)
        assert not torch.equal(out.F, out2.F)


def test_hashfly_equals_precomputed(device):
    # The forward accumulates each row's offsets in the same order in both algorithms, so
    # it agrees bitwise.  The submanifold input gradient of the precomputed path walks the
    # offsets in reverse (it reads the map's symmetric transpose) and the weight gradients
    # sum pairs in different fixed orders: both agree to fp32 rounding.
    rng = np.random.default_rng(21)
    c = _rand_coords(rng, 6000, 24)
    X = rng.standard_normal((6000, 32)).astype(np.float32)
    W = (rng.standard_normal((27, 32, 32)) / 30).astype(np.float32)
    dY = rng.standard_normal((6000, 32)).astype(np.float32)
    res = [_run(device, c, (24, 24, 24), X, W, dY, 3, 1, 1, 1, False, True, torch.float32, a) for a in ConvAlgo]
    assert torch.equal(res[0][0].F, res[1][0].F)
    assert rel(res[0][1].cpu(), res[1][1].cpu()) < 1e-6
    assert rel(res[0][2].cpu(), res[1][2].cpu()) < 1e-6


@pytest.mark.parametrize("case", ["in_box", "out_of_box", "duplicates", "both"])
@pytest.mark.parametrize("cin,cout,dtype,d", [(64, 64, torch.bfloat16, 1), (128, 128, torch.bfloat16, 1),
                                              (64, 128, torch.float32, 1), (128, 64, torch.float16, 1),
                                              (64, 64, torch.float32, 2)])
def test_subm_brick_fly_path(device, case, cin, cout, dtype, d):
    """Hash-fly submanifold convolutions at built shapes look neighbours up in the brick index
    inside the GEMM (ConvSubmFlyGEMM).  Forward, dX and dW against the float64 oracle; the
    forward and the weight gradient bitwise equal to the precomputed path (same per-row
    offset order, same pair list); the input gradient through the reversed-weight fly GEMM
    (unique coordinates in the box) or the transposed map queried from the index."""
    from sparsetriton_amd.nn.functional.conv.kmap import BrickIndex
    rng = np.random.default_rng(37 + cin + d)
    n, S = 3000, 20
    c = _rand_coords(rng, n, S)
    shape = (S, S, S)
    if case in ("out_of_box", "both"):
        shape = (15, 18, 20)
    if case in ("duplicates", "both"):
        rows = rng.choice(n, 150, replace=False)
        c[rows[75:]] = c[rows[:75]]
    X = rng.standard_normal((n, cin)).astype(np.float32)
    W = (rng.standard_normal((27, cin, cout)) / np.sqrt(27 * cin)).astype(np.float32)
    dY = rng.standard_normal((n, cout)).astype(np.float32)
    res = {}
    for algo in ConvAlgo:
        set_conv_algo(algo)
        feats = torch.as_tensor(X, device=device).to(dtype).requires_grad_(True)
        w = torch.as_tensor(W, device=device).to(dtype).requires_grad_(True)
        sp = SparseTensor(feats, torch.as_tensor(c, device=device), spatial_shape=shape, batch_size=2)
        out = sparse_conv3d(sp, w, 3, dilation=d)
        out.F.backward(torch.as_tensor(dY, device=device).to(dtype))
        res[algo] = (out.F.detach(), feats.grad, w.grad)
        if algo == ConvAlgo.ImplicitHashFlyGEMM:
            index = sp._cache.kmaps[("brick_index", 2, shape)]
            assert isinstance(index, BrickIndex)  # the fly path ran
            assert index.transposable() == (case == "in_box")
    set_conv_algo(ConvAlgo.PrecomputedNeighborGEMM)
    fly, pre = res[ConvAlgo.ImplicitHashFlyGEMM], res[ConvAlgo.PrecomputedNeighborGEMM]
    assert torch.equal(fly[0], pre[0])
    assert torch.equal(fly[2], pre[2])
    Xq = torch.as_tensor(X).to(dtype).float().numpy()
    Wq = torch.as_tensor(W).to(dtype).float().numpy()
    dYq = torch.as_tensor(dY).to(dtype).float().numpy()
    y, gx, gw = _oracle(c, c, shape, Xq, Wq, dYq, 3, 1, d, d, False)
    tol = TOL[dtype]
    assert rel(fly[0].float().cpu(), y) < tol
    assert rel(fly[1].float().cpu(), gx) < tol, case
    assert rel(fly[2].float().cpu(), gw) < tol
    assert rel(fly[1].float().cpu(), pre[1].float().cpu()) < tol / 4


def test_brick_index_query_equals_subm_map(device):
    """st_subm_index + st_kmap_subm_query give st_kmap_subm's map and masks; the index's status
    words count the same duplicates and out-of-box rows."""
    from sparsetriton_amd.nn.functional.conv.kmap import BrickIndex, _target_offsets, subm_kernel_map
    rng = np.random.default_rng(38)
    c = _rand_coords(rng, 5000, 24)
    c[:40] = c[40:80]
    coords = torch.as_tensor(c, device=device)
    for shape, d in (((24, 24, 24), 1), ((20, 24, 22), 2)):
        offs = _target_offsets(3, d, d, False, device)
        km, snap = subm_kernel_map(coords, 2, shape, offs, symmetric=False)
        index = BrickIndex.build(coords, 2, shape)
        q = index.query(offs)
        assert torch.equal(q.nbr, km.nbr) and torch.equal(q.out_masks, km.out_masks)
        assert index.status.counters() == snap.counters()
        if shape == (24, 24, 24):  # (repeats outside a smaller box are not indexed, so not counted)
            assert snap.counters()["duplicate"] == 40 and snap.counters()["out_of_box"] == 0
        # the masks-only query (nbr = NULL) behind the fly GEMMs' tile order: the same mask words
        from sparsetriton_amd import _lib
        mo = torch.full_like(q.out_masks, -7)
        _lib.call("st_kmap_subm_query", _lib.ptr(coords), _lib.coord_code(coords.dtype), coords.shape[0],
                  _lib.ptr(offs), offs.shape[0], *index.geometry, _lib.ptr(index.work), index.nbytes, None,
                  _lib.ptr(mo), _lib.stream_of(coords.device))
        assert torch.equal(mo, q.out_masks)
        order = index.tile_order(offs, ("t", d))
        n = coords.shape[0]
        assert torch.equal(torch.sort(order.long())[0].cpu(), torch.arange(n))
        key = km.out_masks[:, 0].long().cpu().numpy()
        o = order.long().cpu().numpy()
        runs = np.flatnonzero(np.diff(key[o])) + 1  # rows of one mask are contiguous in the order
        assert len(np.unique(key)) == len(runs) + 1


@pytest.mark.parametrize("cin,cout,dtype", [(64, 64, torch.bfloat16), (128, 128, torch.bfloat16),
                                            (64, 128, torch.float32), (128, 64, torch.float16)])
def test_subm_fly_tile_order_and_reversed_offsets(device, cin, cout, dtype):
    """st_subm_fly_gemm over the index's mask-sorted tile order gives the row-order result bit for
    bit (a row's sum does not depend on its tile), and its ST_GATHER_REVERSE_K input gradient with
    the weights as given equals the same call with an ST_W_REVERSE copy, bit for bit."""
    from sparsetriton_amd import _lib
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_hashfly_gemm import subm_fly_gemm
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import weight_prep
    from sparsetriton_amd.nn.functional.conv.kmap import BrickIndex, _target_offsets
    rng = np.random.default_rng(39 + cin)
    n, S = 7000, 22
    c = _rand_coords(rng, n, S)
    shape = (S, S, S)
    coords = torch.as_tensor(c, device=device)
    index = BrickIndex.build(coords, 2, shape)
    assert index.transposable()
    offs = _target_offsets(3, 1, 1, False, device)
    order = index.tile_order(offs, (3, 1, 1))
    assert index.tile_order(offs, (3, 1, 1)) is order  # kept with the index
    X = torch.as_tensor(rng.standard_normal((n, cin)), device=device).to(dtype)
    dY = torch.as_tensor(rng.standard_normal((n, cout)), device=device).to(dtype)
    W = torch.as_tensor(rng.standard_normal((27, cin, cout)) / np.sqrt(27 * cin), device=device).to(dtype)
    wt = weight_prep(W.contiguous(), _lib.W_TRANSPOSE)
    y0 = subm_fly_gemm(X, index, offs, wt)
    y1 = subm_fly_gemm(X, index, offs, wt, order)
    assert torch.equal(y0, y1)
    g0 = subm_fly_gemm(dY, index, offs, weight_prep(W.contiguous(), _lib.W_REVERSE))
    g1 = subm_fly_gemm(dY, index, offs, W.contiguous(), order, reverse_k=True)
    g2 = subm_fly_gemm(dY, index, offs, W.contiguous(), None, reverse_k=True)
    assert torch.equal(g0, g1) and torch.equal(g0, g2)
    # against the float64 oracle's input gradient of the same map
    Xq, Wq, dYq = X.float().cpu().numpy(), W.float().cpu().numpy(), dY.float().cpu().numpy()
    y, gx, _ = _oracle(c, c, shape, Xq, Wq, dYq, 3, 1, 1, 1, False)
    assert rel(y1.float().cpu(), y) < TOL[dtype]
    assert rel(g1.float().cpu(), gx) < TOL[dtype]

@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_probing_weight_gradient_entry(device, dtype, tol):
    """st_hashfly_wgrad, which probes the table inside the weight-gradient kernel (the autograd
    path probes once into a pair list instead), against the oracle."""
    from sparsetriton_amd.nn.functional.conv.conv import _input_table
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_hashfly_gemm import _lookup, hashfly_wgrad_probing
    from sparsetriton_amd.nn.functional.conv.kmap import _target_offsets
    rng = np.random.default_rng(24)
    c = _rand_coords(rng, 3000, 20)
    X = rng.standard_normal((3000, 32)).astype(np.float32)
    dY = rng.standard_normal((3000, 16)).astype(np.float32)
    sp = SparseTensor(torch.as_tensor(X, device=device), torch.as_tensor(c, device=device),
                      spatial_shape=(20, 20, 20), batch_size=2)
    table = _input_table(sp, 1)
    offs = _target_offsets(3, 1, 1, False, device).to(torch.int32).contiguous()
    dW = hashfly_wgrad_probing(sp.F.to(dtype), torch.as_tensor(dY, device=device).to(dtype), sp.C, offs,
                               _lookup(27, -1, 1, 1, (20, 20, 20)), table.table_keys, table.table_values,
                               torch.float32)
    Xr = torch.as_tensor(X).to(dtype).double().numpy()
    dYr = torch.as_tensor(dY).to(dtype).double().numpy()
    nbr = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, (20, 20, 20))
    assert rel(dW.cpu(), O.wgrad_f64(Xr, dYr, nbr, 27)) < tol


def test_deterministic(device):
    rng = np.random.default_rng(22)
    c = _rand_coords(rng, 8000, 24)
    X = rng.standard_normal((8000, 64)).astype(np.float32)
    W = (rng.standard_normal((27, 64, 64)) / 40).astype(np.float32)
    dY = rng.standard_normal((8000, 64)).astype(np.float32)
    r1 = _run(device, c, (24, 24, 24), X, W, dY, 3, 1, 1, 1, False, True, torch.bfloat16,
              ConvAlgo.PrecomputedNeighborGEMM)
    r2 = _run(device, c, (24, 24, 24), X, W, dY, 3, 1, 1, 1, False, True, torch.bfloat16,
              ConvAlgo.PrecomputedNeighborGEMM)
    assert torch.equal(r1[0].F, r2[0].F) and torch.equal(r1[1], r2[1]) and torch.equal(r1[2], r2[2])


def test_plain_neighbor_indices_tensor(device):
    # ConvPrecomputedNeighborGEMM.apply with the reference's (N_out, K) tensor form
    from sparsetriton_amd.nn.functional.conv.funcs import ConvPrecomputedNeighborGEMM
    rng = np.random.default_rng(23)
    c = _rand_coords(rng, 3000, 20)
    nbr = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, (20, 20, 20))
    X = rng.standard_normal((3000, 16)).astype(np.float32)
    W = (rng.standard_normal((27, 16, 24)) / 20).astype(np.float32)
    dY = rng.standard_normal((3000, 24)).astype(np.float32)
    feats = torch.as_tensor(X, device=device).requires_grad_(True)
    w = torch.as_tensor(W, device=device).requires_grad_(True)
    out = ConvPrecomputedNeighborGEMM.apply(feats, w, torch.as_tensor(nbr, device=device))
    out.backward(torch.as_tensor(dY, device=device))
    assert rel(out.detach().cpu(), O.fwd_f64(X, W, nbr)) < 1e-5
    assert rel(feats.grad.cpu(), O.dgrad_f64(dY, W, nbr, 3000)) < 1e-5
    assert rel(w.grad.cpu(), O.wgrad_f64(X, dY, nbr, 27)) < 1e-5


def test_plain_map_with_one_input_to_two_outputs(device):
    """A caller's map where an (input, offset) feeds two outputs: the forward is fine; the gather
    input gradient cannot represent it and says so instead of dropping a term."""
    from sparsetriton_amd.nn.functional.conv.funcs import ConvPrecomputedNeighborGEMM
    nbr = torch.full((4, 27), -1, dtype=torch.int32)
    nbr[0, 3] = nbr[2, 3] = 1  # input 1 feeds outputs 0 and 2 through offset 3
    nbr[1, 13] = 0
    g = torch.Generator(device="cpu").manual_seed(0)
    feats = torch.randn(2, 8, generator=g).to(device).requires_grad_(True)
    w = torch.randn(27, 8, 8, generator=g).to(device).requires_grad_(True)
    out = ConvPrecomputedNeighborGEMM.apply(feats, w, nbr.to(device))
    ref = O.fwd_f64(feats.detach().cpu().numpy(), w.detach().cpu().numpy(), nbr.numpy())
    assert rel(out.detach().cpu(), ref) < 1e-4
    with pytest.raises(ValueError, match="several output rows"):
        out.sum().backward()


# --------------------------------------------- reference test parametrisations

@pytest.mark.parametrize("C_in,C_out,k,s,p,d", [(8, 16, 3, 1, 1, 1), (4, 8, 3, 2, 1, 1), (16, 16, 5, 2, 2, 1),
                                                (16, 16, 5, 1, 2, 1)])
def test_reference_forward_vs_dense(device, C_in, C_out, k, s, p, d):
    torch.manual_seed(0)
    sp = randn((10, 10, 10), batch_size=1, channels=C_in, nnz=27, device=device).half()
    weight = torch.rand(k ** 3, C_in, C_out, device=device, dtype=torch.float16)
    st_out = sparse_conv3d(sp, weight, kernel_size=k, stride=s, padding=p, dilation=d, submanifold=False).float()
    w_t = weight.view(k, k, k, C_in, C_out).permute(4, 3, 0, 1, 2).contiguous().float().cpu()
    dense_in = sp.dense().permute(0, 4, 1, 2, 3).contiguous().float().cpu()
    dense_out = torch.nn.functional.conv3d(dense_in, w_t, stride=s, padding=p, dilation=d)
    st_dense = st_out.dense().cpu()
    torch.testing.assert_close(st_dense, dense_out.permute(0, 2, 3, 4, 1).contiguous(), atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("C_in,C_out,k,s,p,d", [(16, 16, 3, 1, 1, 1), (32, 32, 3, 1, 1, 1), (32, 32, 5, 1, 2, 1),
                                                (4, 8, 3, 2, 1, 1), (8, 16, 3, 2, 1, 1), (8, 16, 3, 4, 1, 1)])
def test_reference_transposed_vs_dense(device, C_in, C_out, k, s, p, d):
    torch.manual_seed(1)
    sp = randn((10, 10, 10), batch_size=1, channels=C_in, nnz=27, device=device).half()
    weight = torch.rand(k ** 3, C_in, C_out, device=device, dtype=torch.float16) / k ** 3
    st_out = sparse_conv3d(sp, weight, kernel_size=k, stride=s, padding=p, dilation=d, submanifold=False,
                           transposed=True).float()
    w_t = weight.view(k, k, k, C_in, C_out).permute(3, 4, 0, 1, 2).contiguous().float().cpu()
    dense_in = sp.dense().permute(0, 4, 1, 2, 3).contiguous().float().cpu()
    dense_out = torch.nn.functional.conv_transpose3d(dense_in, w_t, stride=s, padding=p, dilation=d)
    st_dense = st_out.dense().cpu()
    torch.testing.assert_close(st_dense, dense_out.permute(0, 2, 3, 4, 1).contiguous(), atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("C_in,C_out,k,s,p,d", [(16, 16, 3, 1, 2, 1), (32, 32, 3, 1, 0, 1), (32, 32, 5, 1, 2, 1),
                                                (16, 16, 3, 2, 1, 1), (16, 16, 3, 2, 1, 2)])
def test_reference_gradients_vs_dense(device, C_in, C_out, k, s, p, d):
    torch.manual_seed(2)
    sp_in = randn((64, 64, 64), batch_size=1, channels=C_in, nnz=32 ** 3, device=device)
    feats = sp_in.F.half().detach().requires_grad_(True)
    sp_in.F = feats
    weight = (torch.randn(k ** 3, C_in, C_out, device=device, dtype=torch.float16) / k ** 3).requires_grad_(True)
    st_out = sparse_conv3d(sp_in, weight, kernel_size=k, stride=s, padding=p, dilation=d, submanifold=False)
    st_out.dense().float().abs().mean().backward()
    w_t = weight.detach().float().view(k, k, k, C_in, C_out).permute(4, 3, 0, 1, 2).contiguous().requires_grad_(True)
    dense_in = sp_in.dense().permute(0, 4, 1, 2, 3).contiguous().detach().float().requires_grad_(True)
    dense_out = torch.nn.functional.conv3d(dense_in, w_t, stride=s, padding=p, dilation=d)
    dense_out.permute(0, 2, 3, 4, 1).contiguous().abs().mean().backward()
    coords = sp_in.coords.long()
    g_in = dense_in.grad.permute(0, 2, 3, 4, 1)[coords[:, 0], coords[:, 1], coords[:, 2], coords[:, 3]]
    g_w = w_t.grad.permute(2, 3, 4, 1, 0).reshape(k ** 3, C_in, C_out)
    torch.testing.assert_close(weight.grad.float(), g_w, atol=5e-2, rtol=5e-2)
    torch.testing.assert_close(feats.grad.float(), g_in, atol=5e-2, rtol=5e-2)


def test_reference_submanifold_vs_dense(device):
    torch.manual_seed(3)
    for C_in, C_out, ks, pad, nnz in [(8, 16, 3, 1, 100), (8, 16, 5, 2, 120)]:
        sp_in = randn((10, 10, 10), batch_size=1, channels=C_in, nnz=nnz, device=device).half()
        weight = torch.rand(ks ** 3, C_in, C_out, device=device, dtype=torch.float16)
        st_out = sparse_conv3d(sp_in, weight, kernel_size=ks, stride=1, padding=pad, dilation=1, submanifold=True)
        assert torch.equal(st_out.coords, sp_in.coords) and st_out.F.shape == (nnz, C_out)
        w_t = weight.view(ks, ks, ks, C_in, C_out).permute(4, 3, 0, 1, 2).contiguous().float().cpu()
        dense = torch.nn.functional.conv3d(sp_in.dense().permute(0, 4, 1, 2, 3).float().cpu(), w_t, padding=pad)
        c = st_out.coords.long().cpu()
        ref = dense.permute(0, 2, 3, 4, 1)[c[:, 0], c[:, 1], c[:, 2], c[:, 3]]
        torch.testing.assert_close(st_out.F.float().cpu(), ref, atol=1e-3, rtol=1e-3)
    # non-centre padding is forced to centre for submanifold (conv.py:120-121)
    out = sparse_conv3d(sp_in, torch.rand(27, 8, 16, device=device, dtype=torch.float16), 3, padding=0,
                        submanifold=True)
    assert torch.isfinite(out.F).all() and out.F.shape[1] == 16


# ------------------------------------------------------------ modules / cache

def test_module_stack_shares_kernel_map(device):
    sp = randn((32, 32, 32), batch_size=2, nnz=5000, channels=16, device=device)
    l1, l2 = SubMConv3D(16, 32, 3).to(device), SubMConv3D(32, 32, 3).to(device)
    y1 = l1(sp)
    y2 = l2(y1)
    assert y1._cache is sp._cache and y2._cache is sp._cache
    # one map for the stack; a submanifold map is built from its brick index, with no hash table
    assert len(sp._cache.neighbor_indices) == 1 and sp._cache.hashtable is None
    down = SparseConv3D(32, 64, 3, stride=2, padding=1).to(device)(y2)
    up = SparseConvTransposed3D(64, 32, 3, stride=2, padding=1).to(device)(down)
    assert down.F.shape[1] == 64 and up.F.shape[1] == 32
    (up.F.sum() + y2.F.sum()).backward()
    assert torch.isfinite(l1.weight.grad).all() and l1.bias.grad.shape == (32,)


def test_empty_tensor(device):
    sp = SparseTensor(torch.empty((0, 8), device=device), torch.empty((0, 4), dtype=torch.int16, device=device),
                      spatial_shape=(8, 8, 8), batch_size=1)
    for conv in (SubMConv3D(8, 4, 3), SparseConv3D(8, 4, 3, stride=2, padding=1),
                 SparseConvTransposed3D(8, 4, 3, stride=2)):
        out = conv.to(device)(sp)
        assert out.F.shape == (0, 4)


# ------------------------------------------------ benchmark-size properties

def test_config2_full_size_properties(device):
    """SubM 64->64 on the full config-2 set: exact rows on a sample, adjoint identities overall."""
    c, shape = workloads.config2()
    n = c.shape[0]
    rng = np.random.default_rng(5)
    X = rng.standard_normal((n, 64)).astype(np.float32)
    W = (rng.standard_normal((27, 64, 64)) / np.sqrt(27 * 64)).astype(np.float32)
    dY = rng.standard_normal((n, 64)).astype(np.float32)
    for dtype, tol in ((torch.float32, 2e-3), (torch.bfloat16, 2e-2)):
        Xq = torch.as_tensor(X).to(dtype)
        Wq = torch.as_tensor(W).to(dtype)
        dYq = torch.as_tensor(dY).to(dtype)
        out, dX, dW = _run(device, c, shape, Xq.float().numpy(), Wq.float().numpy(), dYq.float().numpy(), 3, 1, 1,
                           1, False, True, dtype, ConvAlgo.PrecomputedNeighborGEMM)
        y = out.F.detach().double().cpu()
        # adjoint identities: <dY, Y> = <dX, X> = <dW, W> (linearity in X and in W)
        s_y = float((dYq.double() * y).sum())
        s_x = float((dX.double().cpu() * Xq.double()).sum())
        s_w = float((dW.double().cpu() * Wq.double()).sum())
        assert abs(s_x - s_y) <= tol * abs(s_y) and abs(s_w - s_y) <= tol * abs(s_y)
        # exact rows on a random sample
        rows = rng.choice(n, 3000, replace=False)
        nbr = O.exact_kmap(c, c[rows], O.target_offsets(3, 1, 1, False), 1, shape)
        y_ref = O.fwd_f64(Xq.float().numpy(), Wq.float().numpy(), nbr)
        assert rel(y[rows].numpy(), y_ref) < tol


# --------------------------------------------------------------- fused bias

@pytest.mark.parametrize("algo", list(ConvAlgo))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cin,cout", [(16, 32), (64, 64), (256, 32), (20, 36)])
def test_bias_vs_oracle(device, algo, dtype, cin, cout):
    """out = conv + bias (the reference's `out_feats += bias`, conv.py:227-228; fused into the
    GEMM's store on the precomputed path, tiled and untiled reductions alike), dbias = sum of dY."""
    rng = np.random.default_rng(cin + 7 * cout)
    c = _rand_coords(rng, 3000, 18)
    X = torch.as_tensor(rng.standard_normal((3000, cin)).astype(np.float32)).to(dtype).float().numpy()
    W = torch.as_tensor((rng.standard_normal((27, cin, cout)) / np.sqrt(27 * cin)).astype(np.float32)).to(dtype)
    b = torch.as_tensor(rng.standard_normal(cout).astype(np.float32)).to(dtype)
    dY = torch.as_tensor(rng.standard_normal((3000, cout)).astype(np.float32)).to(dtype).float().numpy()
    set_conv_algo(algo)
    feats = torch.as_tensor(X, device=device).to(dtype).requires_grad_(True)
    w = W.to(device).requires_grad_(True)
    bias = b.to(device).requires_grad_(True)
    sp = SparseTensor(feats, torch.as_tensor(c, device=device), spatial_shape=(18, 18, 18))
    out = sparse_conv3d(sp, w, 3, bias=bias)
    out.F.backward(torch.as_tensor(dY, device=device).to(dtype))
    y, gx, gw = _oracle(c, c, (18, 18, 18), X, W.float().numpy(), dY, 3, 1, 1, 1, False)
    y = y + b.float().numpy()[None, :]
    tol = TOL[dtype]
    assert rel(out.F.detach().float().cpu(), y) < tol
    assert rel(feats.grad.float().cpu(), gx) < tol
    assert rel(w.grad.float().cpu(), gw) < tol
    assert bias.grad.dtype == dtype
    assert rel(bias.grad.float().cpu(), dY.sum(0)) < tol


def test_bias_without_sources(device):
    """A gather with no source rows stores the bias broadcast over its rows."""
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import gather_gemm, gather_gemm_tiled
    from sparsetriton_amd.nn.functional.conv.kmap import TileMap, TilePlan
    K, n_dst = 27, 300
    nbr = torch.full((K, n_dst), -1, dtype=torch.int32, device=device)
    masks = torch.zeros((n_dst, 1), dtype=torch.int32, device=device)
    perm = TilePlan.build(n_dst, K, masks).perm
    tiles = TileMap.build(nbr, n_dst, 1, masks, K, perm, n_dst, 0)
    for dt in (torch.float32, torch.bfloat16):
        A = torch.empty((0, 64), dtype=dt, device=device)
        Bt = torch.randn((K, 48, 64), device=device).to(dt)
        b = torch.randn(48, device=device).to(dt)
        for out in (gather_gemm_tiled(A, tiles, Bt, n_dst, K, bias=b),
                    gather_gemm(A, nbr, n_dst, 1, masks, Bt, n_dst, K, bias=b)):
            assert torch.equal(out, b[None, :].expand(n_dst, 48))


@pytest.mark.parametrize("n,C", [(0, 16), (1, 7), (1000, 64), (470_532, 64), (3001, 300), (50_000, 128)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_column_sum(device, n, C, dtype):
    """st_column_sum (the bias gradient) against a float64 sum, and bitwise repeatable."""
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import column_sum
    Y = torch.randn((n, C), device=device).to(dtype)
    s = column_sum(Y, torch.float32)
    ref = Y.double().sum(0).cpu()
    err = (s.double().cpu() - ref).abs().max().item() if n else s.abs().max().item()
    assert err <= 1e-5 * max(1.0, n ** 0.5) * 4
    assert torch.equal(s, column_sum(Y, torch.float32))
    assert column_sum(Y, dtype).dtype == dtype


# ------------------------------------------------------------- store epilogue

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cin,cout", [(16, 32), (64, 64), (128, 128), (32, 48)])
@pytest.mark.parametrize("s", [1, 2])
def test_fused_epilogue_vs_oracle(device, dtype, cin, cout, s):
    """act((conv + bias) * scale + shift + residual) in the GEMM store vs the float64 oracle."""
    from sparsetriton_amd.nn.functional import sparse_conv3d_fused

    rng = np.random.default_rng(cin * 10 + cout + s)
    S = 16
    c = _rand_coords(rng, 1500, S)
    X = rng.standard_normal((c.shape[0], cin))
    W = rng.standard_normal((27, cin, cout)) / np.sqrt(27 * cin)
    bias = rng.standard_normal(cout)
    scale = rng.uniform(0.5, 1.5, cout)
    shift = rng.standard_normal(cout)
    set_conv_algo(ConvAlgo.PrecomputedNeighborGEMM)
    feats = torch.as_tensor(X, device=device).to(dtype)
    w = torch.as_tensor(W, device=device).to(dtype)
    b = torch.as_tensor(bias, device=device).to(dtype)
    sp = SparseTensor(feats, torch.as_tensor(c, device=device), spatial_shape=(S, S, S))
    with torch.no_grad():
        plain = sparse_conv3d(sp, w, 3, bias=b, stride=s, padding=1, submanifold=(s == 1))
        n_out = plain.F.shape[0]
        res = torch.as_tensor(rng.standard_normal((n_out, cout)), device=device).to(dtype)
        sc = torch.as_tensor(scale, device=device, dtype=torch.float32)
        sh = torch.as_tensor(shift, device=device, dtype=torch.float32)
        out = sparse_conv3d_fused(sp, w, 3, bias=b, stride=s, padding=1, submanifold=(s == 1), scale=sc, shift=sh,
                                  residual=res, relu=True)
        only_relu = sparse_conv3d_fused(sp, w, 3, bias=b, stride=s, padding=1, submanifold=(s == 1), relu=True)
    assert torch.equal(out.C, plain.C)
    oc = out.C.cpu().numpy()
    Xq = feats.double().cpu().numpy()
    Wq = w.double().cpu().numpy()
    off = O.target_offsets(3, 1, 1, False)
    nbr = O.exact_kmap(c, oc, off, s, (S, S, S))
    y = O.fwd_f64(Xq, Wq, nbr) + b.double().cpu().numpy()
    ref = np.maximum(y * scale + shift + res.double().cpu().numpy(), 0.0)
    assert rel(out.F.double().cpu(), ref) < TOL[dtype]
    assert rel(only_relu.F.double().cpu(), np.maximum(y, 0.0)) < TOL[dtype]
    # without an affine map or ReLU the epilogue is the plain bias store, bit for bit
    with torch.no_grad():
        same = sparse_conv3d_fused(sp, w, 3, bias=b, stride=s, padding=1, submanifold=(s == 1))
    assert torch.equal(same.F, plain.F)


def test_fused_epilogue_without_sources(device):
    """No source rows: every output row is the epilogue of a zero sum."""
    import ctypes
    from sparsetriton_amd import _lib

    n_dst, Nd, K, Kd = 300, 32, 27, 16
    dev = device
    perm = torch.arange(n_dst, dtype=torch.int32, device=dev)
    dummy_i32 = torch.zeros(64, dtype=torch.int32, device=dev)
    dummy_i16 = torch.zeros(64, dtype=torch.int16, device=dev)
    Bt = torch.zeros((K, Nd, Kd), dtype=torch.float32, device=dev)
    bias = torch.randn(Nd, device=dev)
    scale = torch.rand(Nd, device=dev) + 0.5
    shift = torch.randn(Nd, device=dev)
    res = torch.randn(n_dst, Nd, device=dev)
    out = torch.empty((n_dst, Nd), device=dev)
    _lib.call("st_gather_gemm_tiled_epilogue", None, 0, _lib.ptr(perm), _lib.ptr(dummy_i32), _lib.ptr(dummy_i16),
              _lib.ptr(dummy_i32), _lib.ptr(Bt), _lib.ptr(bias), _lib.ptr(scale), _lib.ptr(shift), _lib.ptr(res), 1,
              _lib.ptr(out), n_dst, K, Kd, Nd, 0, _lib.stream_of(dev))
    ref = torch.relu(bias * scale + shift + res)
    assert torch.allclose(out, ref, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype,C", [(torch.float32, 64), (torch.bfloat16, 64), (torch.float16, 32),
                                     (torch.bfloat16, 128), (torch.float32, 128)])
def test_reverse_k_gather_equals_reversed_weights(device, dtype, C):
    """The input gradient of a symmetric submanifold map over the forward's plan with the weights'
    offsets reversed as the GEMM addresses them (ST_GATHER_REVERSE_K) equals the same gather over
    an ST_W_REVERSE copy of the weights, bit for bit (ring kernels at 32 / 64 channels, the wide
    kernel at 128 x 128 16-bit and 64 x 128 split fp32)."""
    from sparsetriton_amd import _lib
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import gather_gemm_tiled, weight_prep
    from sparsetriton_amd.nn.functional.conv.kmap import _target_offsets, subm_kernel_map
    rng = np.random.default_rng(C + 3)
    c = _rand_coords(rng, 6000, 24)
    coords = torch.as_tensor(c, device=device)
    km, _ = subm_kernel_map(coords, 2, (24, 24, 24), _target_offsets(3, 1, 1, False, device))
    assert km.symmetric
    cout = 64 if C == 128 and dtype == torch.float32 else C
    dY = torch.randn((6000, cout), device=device).to(dtype)
    W = (torch.randn((27, C, cout), device=device) / 40).to(dtype)
    tiles = km.backward_tiles()
    a = gather_gemm_tiled(dY, tiles, W, km.n_in, 27, reverse_k=True)
    b = gather_gemm_tiled(dY, tiles, weight_prep(W, _lib.W_REVERSE), km.n_in, 27)
    assert torch.equal(a, b)
    ref = O.dgrad_f64(dY.float().cpu().numpy(), W.float().cpu().numpy(), km.neighbor_indices.cpu().numpy(), 6000)
    assert rel(a.float().cpu().numpy(), ref) < TOL[dtype]
