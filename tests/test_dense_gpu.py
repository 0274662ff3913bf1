"""to_dense / its gradient (st_to_dense / st_from_dense) on the GPU.

Pinned by the reference's known answer (utils/to_dense.py:259-270), by a
brute-force loop over the rows for random sets (every dtype and coordinate
dtype, channel counts on and off the 16-byte vector path), by the gradient
being the gather at the same cells, and by out-of-grid coordinates being
skipped.
"""

import numpy as np
import pytest
import torch

from sparsetriton_amd import SparseTensor
from sparsetriton_amd.utils import to_dense

pytestmark = pytest.mark.gpu


def test_dense_layout_kat(device):
    feats = torch.tensor([[1.0], [2.0], [3.0]], device=device)
    coords = torch.tensor([[0, 0, 0, 0], [0, 0, 0, 1], [1, 0, 0, 0]], device=device)
    d = to_dense(feats, coords, (1, 1, 2))
    assert d.shape == (2, 1, 1, 2, 1)
    assert d[0, 0, 0, 0, 0] == 1.0 and d[0, 0, 0, 1, 0] == 2.0 and d[1, 0, 0, 0, 0] == 3.0
    assert float(d.sum()) == 6.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("C", [1, 3, 8, 64])
@pytest.mark.parametrize("cdt", [torch.int16, torch.int32, torch.int64])
def test_to_dense_vs_loop(device, dtype, C, cdt):
    rng = np.random.default_rng(C)
    B, S = 3, (7, 5, 9)
    lin = rng.choice(B * S[0] * S[1] * S[2], 150, replace=False)
    b, r = np.divmod(lin, S[0] * S[1] * S[2])
    x, r = np.divmod(r, S[1] * S[2])
    y, z = np.divmod(r, S[2])
    coords = np.stack([b, x, y, z], 1)
    B = int(coords[:, 0].max()) + 1  # the grid's batch extent (max index + 1)
    f = torch.randn(len(lin), C).to(dtype).to(device).requires_grad_(True)
    ct = torch.as_tensor(coords, device=device).to(cdt)
    d = to_dense(f, ct, S)
    ref = torch.zeros((B,) + S + (C,), dtype=dtype)
    fc = f.detach().cpu()
    for i, (bb, xx, yy, zz) in enumerate(coords.tolist()):
        ref[bb, xx, yy, zz] = fc[i]
    assert torch.equal(d.cpu(), ref)
    g = torch.randn(d.shape).to(dtype).to(device)
    d.backward(g)
    gc = g.cpu()
    expect = torch.stack([gc[bb, xx, yy, zz] for bb, xx, yy, zz in coords.tolist()])
    assert torch.equal(f.grad.cpu(), expect)


def test_out_of_grid_skipped(device):
    feats = torch.ones(3, 4, device=device)
    coords = torch.tensor([[0, 0, 0, 0], [0, 5, 0, 0], [0, 1, 1, 1]], device=device, dtype=torch.int32)
    d = to_dense(feats, coords, (2, 2, 2))
    assert float(d.sum()) == 8.0 and d[0, 1, 1, 1, 0] == 1.0


def test_sparse_tensor_dense(device):
    sp = SparseTensor(torch.arange(6.0, device=device).view(3, 2),
                      torch.tensor([[0, 1, 2, 3], [1, 0, 0, 0], [0, 3, 3, 3]], device=device))
    d = sp.dense()
    assert d.shape == (2, 4, 4, 4, 2)
    assert d[0, 1, 2, 3].tolist() == [0.0, 1.0] and d[0, 3, 3, 3].tolist() == [4.0, 5.0]


@pytest.mark.parametrize("cdt", [torch.int16, torch.int32, torch.int64])
def test_mask_spatial_range(device, cdt):
    from sparsetriton_amd.utils import mask_spatial_range

    rng = np.random.default_rng(3)
    c = rng.integers(-5, 20, (1000, 4))
    ct = torch.as_tensor(c, device=device).to(cdt)
    m = mask_spatial_range(ct, (0, 9), (2, None), (None, 15)).cpu().numpy()
    ref = (c[:, 1] >= 0) & (c[:, 1] <= 9) & (c[:, 2] >= 2) & (c[:, 3] <= 15)
    assert (m == ref).all()
    assert mask_spatial_range(ct).all()
    assert mask_spatial_range(ct[:0]).shape == (0,)
