"""Weight gradient over windows of output rows (``st_wgrad`` with 16-bit rows and channel counts
that are multiples of 128): dW[k] = sum over the map's pairs (i, o) of offset k of X[i]^T dY[o]
(implicit_precomputed_gemm.py:180-230), checked against the float64 oracle on random maps of
every density, offset count, window count, channel tiling and map layout, and on rows whose dY
holds non-finite values (they may reach only the offsets that pair them)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from sparsetriton_amd import _lib

pytestmark = pytest.mark.gpu


def _map(rng, n_out, n_in, K, density):
    nbr = rng.integers(0, max(n_in, 1), size=(n_out, K)).astype(np.int32)
    nbr[rng.random((n_out, K)) >= density] = -1
    return nbr


def _st_wgrad(X, dY, nbr_dev, ks, rs, n_out, K, splits, dw_dtype=torch.float32, rows=None):
    C_in, C_out = X.shape[1], dY.shape[1]
    partials = torch.empty((K * splits * C_in * C_out,), dtype=torch.float32, device=X.device)
    dW = torch.empty((K, C_in, C_out), dtype=dw_dtype, device=X.device)
    _lib.call("st_wgrad", _lib.ptr(X), X.shape[0], _lib.ptr(dY), _lib.ptr(nbr_dev), ks, rs,
              None if rows is None else _lib.ptr(rows), n_out, K, C_in, C_out,
              _lib.feat_code(X.dtype), _lib.ptr(partials), splits, _lib.ptr(dW), _lib.feat_code(dw_dtype),
              _lib.stream_of(X.device))
    return dW


def _to_dev(nbr, layout, device):
    """The (N_out, K) map on the device as (tensor, k_stride, r_stride): layout "kn" stores it
    offset-major (K, N_out), "nk" row-major."""
    if layout == "kn":
        return torch.from_numpy(np.ascontiguousarray(nbr.T)).to(device), nbr.shape[0], 1
    return torch.from_numpy(np.ascontiguousarray(nbr)).to(device), 1, nbr.shape[1]


CASES = [
    # n_out, n_in, K, density, C_in, C_out, splits, layout, dtype
    (1, 7, 27, 1.0, 128, 128, 1, "kn", torch.bfloat16),
    (31, 40, 27, 0.7, 128, 128, 1, "kn", torch.bfloat16),
    (32, 40, 27, 0.7, 128, 128, 2, "kn", torch.float16),
    (33, 40, 27, 0.7, 128, 128, 3, "nk", torch.bfloat16),
    (1000, 900, 27, 0.67, 128, 128, 5, "kn", torch.bfloat16),
    (5003, 4000, 27, 0.3, 128, 128, 36, "kn", torch.bfloat16),
    (5003, 6100, 27, 0.05, 128, 128, 7, "nk", torch.float16),
    (2000, 2500, 1, 0.9, 128, 128, 4, "kn", torch.bfloat16),
    (2000, 2500, 3, 0.5, 128, 128, 4, "kn", torch.bfloat16),
    (2000, 2500, 4, 0.5, 128, 128, 4, "kn", torch.bfloat16),
    (2000, 2500, 5, 0.5, 128, 128, 4, "kn", torch.bfloat16),
    (2000, 2500, 8, 0.6, 256, 128, 3, "kn", torch.bfloat16),
    (2000, 2500, 8, 0.6, 128, 256, 3, "nk", torch.float16),
    (1500, 1200, 27, 0.5, 256, 256, 2, "kn", torch.bfloat16),
    (3000, 3500, 125, 0.2, 128, 128, 3, "kn", torch.bfloat16),
    (100, 90, 27, 0.5, 128, 128, 300, "kn", torch.bfloat16),   # windows past the rows: zero partials
    (4000, 4000, 27, 0.0, 128, 128, 8, "kn", torch.bfloat16),  # no pairs at all
]


@pytest.mark.parametrize("n_out,n_in,K,density,C_in,C_out,splits,layout,dtype", CASES)
def test_window_wgrad_matches_oracle(device, n_out, n_in, K, density, C_in, C_out, splits, layout, dtype):
    rng = np.random.default_rng(n_out * 131 + K * 7 + C_in + splits)
    nbr = _map(rng, n_out, n_in, K, density)
    X = torch.randn(n_in, C_in, dtype=dtype, device=device)
    dY = torch.randn(n_out, C_out, dtype=dtype, device=device)
    m, ks, rs = _to_dev(nbr, layout, device)
    dW = _st_wgrad(X, dY, m, ks, rs, n_out, K, splits)
    ref = O.wgrad_f64_blas(X.float().cpu().numpy(), dY.float().cpu().numpy(), nbr, K)
    got = dW.cpu().numpy().astype(np.float64)
    # bf16 / fp16 products are exact in fp32; what is left is fp32 summation over <= n_out terms
    scale = np.abs(X.float().cpu().numpy()).max() * np.abs(dY.float().cpu().numpy()).max() if n_out else 1.0
    tol = 1e-6 * scale * max(1, n_out) ** 0.5 * 8
    assert np.abs(got - ref).max() <= tol + 1e-12, (np.abs(got - ref).max(), tol)
    if density == 0.0:
        assert not got.any()


def test_window_wgrad_bf16_output_and_repeat(device):
    """dW in bf16 (the reduce rounds once) and a second call on the same buffers' shapes."""
    rng = np.random.default_rng(5)
    for n_out in (3000, 1700):
        nbr = _map(rng, n_out, 2000, 27, 0.6)
        X = torch.randn(2000, 128, dtype=torch.bfloat16, device=device)
        dY = torch.randn(n_out, 128, dtype=torch.bfloat16, device=device)
        m, ks, rs = _to_dev(nbr, "kn", device)
        dW = _st_wgrad(X, dY, m, ks, rs, n_out, 27, 6, dw_dtype=torch.bfloat16)
        ref = O.wgrad_f64_blas(X.float().cpu().numpy(), dY.float().cpu().numpy(), nbr, 27)
        got = dW.float().cpu().numpy()
        assert np.abs(got - ref).max() <= 2 ** -7 * np.abs(ref).max() + 1e-3


def test_window_wgrad_non_finite_rows_stay_in_their_offsets(device):
    """A dY row holding inf / nan reaches dW[k] only through the offsets that pair it: the window
    kernel multiplies every step's 32 dY rows against each offset's X rows, zeros where the map
    has no pair, and must not let 0 * inf = nan into the offsets without one."""
    rng = np.random.default_rng(11)
    n, K = 2000, 27
    nbr = _map(rng, n, n, K, 0.5)
    bad = [37, 38, 1500]
    nbr[bad, :] = -1
    nbr[37, 4] = 12          # row 37 pairs through offset 4 only
    nbr[38, 20] = 99         # row 38 through offset 20 only; row 1500 through none
    X = torch.randn(n, 128, dtype=torch.bfloat16, device=device)
    dYc = torch.randn(n, 128, dtype=torch.float32)
    dYc[37, 5] = float("inf")
    dYc[38, :] = float("nan")
    dYc[1500, :] = float("-inf")
    dY = dYc.to(torch.bfloat16).to(device)
    m, ks, rs = _to_dev(nbr, "kn", device)
    got = _st_wgrad(X, dY, m, ks, rs, n, K, 4).cpu().numpy().astype(np.float64)
    Xn, dYn = X.float().cpu().numpy(), dY.float().cpu().numpy()
    clean = nbr.copy()
    clean[bad, :] = -1
    ref = O.wgrad_f64_blas(Xn, dYn, clean, K)
    for k in range(K):
        if k in (4, 20):
            continue
        assert np.isfinite(got[k]).all(), k
        assert np.abs(got[k] - ref[k]).max() <= 1e-3, k
    # offset 4: column 5 gets X[12] * inf (+-inf), the other columns stay finite
    assert np.isfinite(np.delete(got[4], 5, axis=1)).all()
    assert not np.isfinite(got[4][:, 5]).any()
    assert np.isnan(got[20]).all()


@pytest.mark.parametrize("order", ["random", "slab-mask", "invalid-entries"])
def test_window_wgrad_column_orders(device, order):
    """The window kernel takes the map's columns in a caller's order: map column p pairs with dY
    row rows[p], so any permutation of the columns (with rows permuted alike) gives the same dW;
    columns whose rows entry lies outside [0, n_out) add nothing."""
    rng = np.random.default_rng({"random": 1, "slab-mask": 2, "invalid-entries": 3}[order])
    n_out, n_in, K = 6000, 5000, 27
    nbr = _map(rng, n_out, n_in, K, 0.6)
    nbr[rng.random(n_out) < 0.3, :13] = -1  # masks that differ between rows
    if order == "slab-mask":
        masks = ((nbr >= 0) * (1 << np.arange(K))).sum(1)
        rows = np.lexsort((masks, np.arange(n_out) // 1024)).astype(np.int32)
    else:
        rows = rng.permutation(n_out).astype(np.int32)
    permuted = nbr[rows]  # column p of the map handed over is row rows[p]'s
    expect_nbr = nbr
    if order == "invalid-entries":
        drop = rng.choice(n_out, 40, replace=False)
        expect_nbr = nbr.copy()
        expect_nbr[rows[drop], :] = -1
        rows[drop[:20]] = -7
        rows[drop[20:]] = n_out + rng.integers(0, 1000, 20)
    X = torch.randn(n_in, 128, dtype=torch.bfloat16, device=device)
    dY = torch.randn(n_out, 128, dtype=torch.bfloat16, device=device)
    m, ks, rs = _to_dev(permuted, "kn", device)
    got = _st_wgrad(X, dY, m, ks, rs, n_out, K, 5, rows=torch.from_numpy(rows).to(device))
    ref = O.wgrad_f64_blas(X.float().cpu().numpy(), dY.float().cpu().numpy(), expect_nbr, K)
    err = np.abs(got.cpu().numpy().astype(np.float64) - ref).max()
    assert err <= 1e-3, err


def test_window_order_of_kernel_map(device):
    """``KernelMap.window_order``: rows sorted by first mask word within slabs (a permutation) and
    the map's columns in that order; the window weight gradient over it equals the plain one."""
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import wgrad_scan
    from sparsetriton_amd.nn.functional.conv.kmap import KernelMap
    rng = np.random.default_rng(9)
    n, K = 5000, 27
    nbr = _map(rng, n, n, K, 0.5)
    km = KernelMap.from_neighbor_indices(torch.from_numpy(nbr).to(device), n)
    rows, m = km.window_order(1024)
    rows_h = rows.cpu().numpy()
    masks = ((nbr >= 0) * (1 << np.arange(K))).sum(1)
    assert np.array_equal(rows_h, np.lexsort((masks, np.arange(n) // 1024)))
    assert np.array_equal(m.cpu().numpy(), nbr[rows_h].T)
    assert km.window_order(1024)[0] is rows
    X = torch.randn(n, 128, dtype=torch.bfloat16, device=device)
    dY = torch.randn(n, 128, dtype=torch.bfloat16, device=device)
    a = wgrad_scan(X, dY, km, torch.float32, splits=3, order=(rows, m)).cpu().numpy()
    b = wgrad_scan(X, dY, km, torch.float32, splits=3).cpu().numpy()
    ref = O.wgrad_f64_blas(X.float().cpu().numpy(), dY.float().cpu().numpy(), nbr, K)
    assert np.abs(a - ref).max() <= 1e-3 and np.abs(b - ref).max() <= 1e-3


def test_column_order_needs_the_window_kernel(device):
    """``rows`` is refused where st_wgrad does not run the window kernel (here 64 channels)."""
    rng = np.random.default_rng(4)
    nbr = _map(rng, 100, 100, 27, 0.5)
    X = torch.randn(100, 64, dtype=torch.bfloat16, device=device)
    dY = torch.randn(100, 64, dtype=torch.bfloat16, device=device)
    m, ks, rs = _to_dev(nbr, "kn", device)
    rows = torch.arange(100, dtype=torch.int32, device=device)
    with pytest.raises(RuntimeError):
        _st_wgrad(X, dY, m, ks, rs, 100, 27, 2, rows=rows)


@pytest.mark.parametrize("concurrent", ["0", "2"])
def test_conv_weight_gradient_through_window_path(device, monkeypatch, concurrent):
    """SubMConv3D 128 -> 128 in bf16 with the weight gradient on the window kernel
    (ST_WGRAD_PATH=window), on the caller's stream and beside the input gradient: dX and dW
    match the float64 oracle, and dW the pair-list path."""
    from sparsetriton_amd import SparseTensor
    from sparsetriton_amd.config import ConvAlgo, set_conv_algo
    from sparsetriton_amd.nn.functional import sparse_conv3d

    rng = np.random.default_rng(21)
    n, S = 6000, 20
    lin = np.sort(rng.choice(2 * S ** 3, n, replace=False))
    c = np.stack([lin // S ** 3, (lin // S ** 2) % S, (lin // S) % S, lin % S], 1).astype(np.int32)
    X = torch.randn(n, 128).to(torch.bfloat16)
    W = (torch.randn(27, 128, 128) / (27 * 128) ** 0.5).to(torch.bfloat16)
    dY = torch.randn(n, 128).to(torch.bfloat16)
    set_conv_algo(ConvAlgo.PrecomputedNeighborGEMM)
    monkeypatch.setenv("ST_CONCURRENT_BACKWARD", concurrent)
    got = {}
    for path in ("window", "pairs"):
        monkeypatch.setenv("ST_WGRAD_PATH", path)
        feats = X.to(device).requires_grad_(True)
        Wd = W.to(device).requires_grad_(True)
        sp = SparseTensor(feats, torch.from_numpy(c).to(device), spatial_shape=(S, S, S))
        out = sparse_conv3d(sp, Wd, 3, submanifold=True)
        out.F.backward(dY.to(device))
        got[path] = (feats.grad.float().cpu().numpy(), Wd.grad.float().cpu().numpy())
    nbr = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, (S, S, S))
    Xn, Wn, dYn = X.float().numpy(), W.float().numpy(), dY.float().numpy()
    gx, gw = O.dgrad_f64(dYn, Wn, nbr, n), O.wgrad_f64_blas(Xn, dYn, nbr, 27)
    for path in got:
        dX, dW = got[path]
        assert np.linalg.norm(dX - gx) <= 2e-2 * np.linalg.norm(gx), path
        assert np.linalg.norm(dW - gw) <= 2e-2 * np.linalg.norm(gw), path
    assert np.abs(got["window"][1] - got["pairs"][1]).max() <= 2 ** -7 * np.abs(got["pairs"][1]).max()
