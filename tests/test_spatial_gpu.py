"""Sparse pooling / upsampling on the GPU vs the float64 oracle (oracle.pool_f64 / upsample_f64).

Output cells and their order are compared exactly; values and gradients as
relative Frobenius errors (fp32 1e-6; bf16 / fp16 round the stored values:
1e-2).  Cases cover odd and even kernels, padding, stride 1..3, negative cells
(even kernel, no padding), unsorted rows, and the reference's own inputs
(tests/test_pooling.py, tests/test_nn_functional.py).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from sparsetriton_amd import SparseTensor, randn
from sparsetriton_amd.nn import SparseDownsample, SparsePooling, SparseUpsample
from sparsetriton_amd.nn.functional import sparse_pooling, sparse_upsample

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-6, torch.bfloat16: 1e-2, torch.float16: 1e-2}


def _np(a):
    if isinstance(a, torch.Tensor):
        return a.detach().double().cpu().numpy()
    return np.asarray(a, dtype=np.float64)


def rel(a, b):
    a, b = _np(a), _np(b)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _set(rng, n, S=10, B=2, shuffle=True):
    lin = rng.choice(B * S ** 3, n, replace=False)
    if not shuffle:
        lin = np.sort(lin)
    return np.stack([lin // S ** 3, (lin // S ** 2) % S, (lin // S) % S, lin % S], 1).astype(np.int32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k,p,s", [(3, 1, 2), (2, 0, 2), (3, 0, 1), (2, 1, 3), (1, 0, 2)])
@pytest.mark.parametrize("mode", ["max", "avg"])
@pytest.mark.parametrize("C", [4, 3, 64])
def test_pooling_vs_oracle(device, dtype, k, p, s, mode, C):
    rng = np.random.default_rng(k * 100 + p * 10 + s + C)
    c = _set(rng, 600)
    x = rng.standard_normal((c.shape[0], C))
    f = torch.as_tensor(x, device=device).to(dtype).requires_grad_(True)
    sp = SparseTensor(f, torch.as_tensor(c, device=device), spatial_shape=(10, 10, 10), batch_size=2)
    out = sparse_pooling(sp, k, p, s, mode)
    xq = _np(f)
    oc, ref, inv = O.pool_f64(c, xq, k, p, s, mode)
    assert np.array_equal(out.C.cpu().numpy().astype(np.int64), oc)
    assert rel(out.F, ref) < TOL[dtype]
    assert tuple(out.spatial_shape) == tuple((10 - k + 2 * p) // s + 1 for _ in range(3))
    dout = rng.standard_normal(tuple(out.F.shape))
    out.F.backward(torch.as_tensor(dout, device=device).to(dtype))
    gref = O.pool_grad_f64(xq, _np(out.F), inv, _np(torch.as_tensor(dout).to(dtype)), mode)
    assert rel(f.grad, gref) < TOL[dtype]


def test_pooling_deterministic_and_negative_cells(device):
    rng = np.random.default_rng(5)
    c = _set(rng, 5000, S=32, B=3)
    sp = SparseTensor(torch.randn(c.shape[0], 16, device=device), torch.as_tensor(c, device=device),
                      spatial_shape=(32, 32, 32), batch_size=3)
    a = sparse_pooling(sp, 2, 0, 2, "avg")
    b = sparse_pooling(sp, 2, 0, 2, "avg")
    assert torch.equal(a.F, b.F) and torch.equal(a.C, b.C)
    # coordinate 0 with an even kernel and no padding lands in cell -1
    assert int(a.C[:, 1:].min()) == -1


def test_reference_pooling_inputs(device):
    # tests/test_pooling.py:57-66 and :96-105: avg pooling / downsampling of tiny sets
    coords = torch.tensor([[0, 0, 0, 0], [0, 0, 0, 1], [0, 0, 1, 0]], dtype=torch.int16, device=device)
    feats = torch.tensor([[1.0], [2.0], [3.0]], device=device)
    sp = SparseTensor(feats, coords, spatial_shape=(2, 2, 2), batch_size=1)
    out = SparsePooling(kernel_size=2, mode="avg", stride=2, padding=0)(sp)
    oc, ref, _ = O.pool_f64(coords.cpu().numpy(), feats.cpu().numpy(), 2, 0, 2, "avg")
    assert isinstance(out, SparseTensor) and np.array_equal(out.C.cpu().numpy(), oc)
    assert torch.allclose(out.F.cpu(), torch.as_tensor(ref, dtype=torch.float32))
    ds = SparseDownsample(scale_factor=2, mode="max")
    assert ds.kernel_size == 2 and ds.stride == 2 and ds.padding == 0
    sp2 = SparseTensor(torch.tensor([[1.0], [2.0]], device=device),
                       torch.tensor([[0, 0, 0, 0], [0, 0, 0, 1]], dtype=torch.int16, device=device),
                       spatial_shape=(4, 4, 4), batch_size=1)
    assert isinstance(ds(sp2), SparseTensor)
    # tests/test_nn_functional.py:42-51 (avg; the reference skips max)
    sp3 = randn((16, 16, 16), batch_size=2, nnz=50, channels=4, device=device)
    for mode in ("avg", "max"):
        out = sparse_pooling(sp3, kernel_size=2, padding=0, stride=2, mode=mode)
        assert isinstance(out, SparseTensor) and out.F.shape[1] == 4


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("scale", [1, 2, 3])
@pytest.mark.parametrize("C", [3, 8])
def test_upsample_vs_oracle(device, dtype, scale, C):
    rng = np.random.default_rng(scale * 10 + C)
    c = _set(rng, 200)
    x = rng.standard_normal((c.shape[0], C))
    f = torch.as_tensor(x, device=device).to(dtype).requires_grad_(True)
    sp = SparseTensor(f, torch.as_tensor(c, device=device), spatial_shape=(10, 10, 10), batch_size=2)
    out = SparseUpsample(scale_factor=scale)(sp)
    oc, of = O.upsample_f64(c, _np(f), scale)
    assert np.array_equal(out.C.cpu().numpy().astype(np.int64), oc)
    assert torch.equal(out.F.detach().cpu(), torch.as_tensor(of).to(dtype))
    assert tuple(out.spatial_shape) == (10 * scale,) * 3
    dout = torch.randn(tuple(out.F.shape), device=device).to(dtype)
    out.F.backward(dout)
    ref = dout.float().view(-1, scale ** 3, C).sum(1)
    assert rel(f.grad, ref) < (1e-6 if dtype == torch.float32 else 1e-2)


def test_upsample_reference_kat(device):
    # tests/test_pooling.py:14-40
    coords = torch.tensor([[0, 0, 0, 0]], dtype=torch.int16, device=device)
    feats = torch.tensor([[1.0, 2.0, 3.0]], device=device)
    sp = SparseTensor(feats, coords, spatial_shape=(10, 10, 10), batch_size=1)
    for s in (1, 2, 3):
        out = sparse_upsample(sp, scale_factor=s)
        assert out.F.shape[0] == s ** 3 and torch.allclose(out.F, feats.repeat(s ** 3, 1))
        expect = [[0, x, y, z] for x in range(s) for y in range(s) for z in range(s)]
        assert out.C.cpu().tolist() == expect
