"""SparseTensor / randn / TensorCache / modules surface (CPU), mirroring the
reference's tests/test_tensor.py and tests/test_nn_modules.py:29-85."""

import pytest
import torch

from sparsetriton_amd import SparseTensor, randn
from sparsetriton_amd.nn import SparseConv3D, SparseConvTransposed3D, SubMConv3D
from sparsetriton_amd.tensor import TensorCache
from sparsetriton_amd.utils import make_ntuple

C3 = torch.tensor([[0, 1, 2, 3], [0, 1, 2, 4], [0, 1, 3, 3]])


def test_init_infers_shape_and_batch():
    sp = SparseTensor(torch.randn(5, 3), torch.tensor([[0, 1, 2, 3], [0, 1, 2, 4], [0, 1, 3, 3], [1, 0, 0, 0],
                                                       [1, 1, 1, 1]]))
    assert sp.spatial_shape == torch.Size([2, 4, 5])
    assert sp.batch_size == 2
    assert sp.coords.dtype == torch.int16


def test_explicit_and_empty():
    assert SparseTensor(torch.randn(3, 4), C3, spatial_shape=(10, 10, 10)).spatial_shape == torch.Size([10, 10, 10])
    assert SparseTensor(torch.randn(3, 4), C3, batch_size=5).batch_size == 5
    sp = SparseTensor(torch.empty(0, 3), torch.empty(0, 4, dtype=torch.int16))
    assert sp.batch_size == 0 and sp.spatial_shape == torch.Size([0, 0, 0])


def test_init_errors():
    with pytest.raises(AssertionError, match="must match"):
        SparseTensor(torch.randn(5, 3), torch.tensor([[0, 1, 2, 3]]))
    with pytest.raises(AssertionError, match="shape .*N, 4.*"):
        SparseTensor(torch.randn(5, 3), torch.randn(5, 3))
    with pytest.raises(AssertionError, match="must be 2D"):
        SparseTensor(torch.randn(5, 3, 2), torch.randn(5, 4))
    with pytest.raises(AssertionError, match="batch_size .* must be >"):
        SparseTensor(torch.randn(3, 4), torch.tensor([[0, 1, 2, 3], [0, 1, 2, 4], [5, 1, 3, 3]]), batch_size=3)


def test_properties_and_methods():
    sp = SparseTensor(torch.randn(3, 4), C3, spatial_shape=(10, 10, 10), batch_size=2)
    assert torch.equal(sp.F, sp.feats) and torch.equal(sp.C, sp.coords)
    sp2 = sp.replace(torch.randn(3, 5))
    assert sp2._cache is sp._cache and sp2.spatial_shape == sp.spatial_shape and sp2.batch_size == 2
    assert sp.half().feats.dtype == torch.float16 and sp.float().feats.dtype == torch.float32
    assert sp.cpu().feats.device.type == "cpu"
    assert "SparseTensor" in repr(sp) and "spatial_shape=" in repr(sp)
    s = sp + sp
    assert torch.allclose(s.F, 2 * sp.F)


def test_randn():
    sp = randn((16, 16, 16), batch_size=2, nnz=100, channels=4)
    assert sp.feats.shape == (100, 4) and torch.unique(sp.coords, dim=0).shape[0] == 100
    assert sp.spatial_shape == torch.Size([16, 16, 16])
    with pytest.raises(ValueError, match="nnz .* exceeds"):
        randn((2, 2, 2), batch_size=1, nnz=10)
    assert randn((2, 2, 2), nnz=1, channels=4).feats.shape == (1, 4)


def test_cache():
    c = TensorCache()
    assert len(c.kmaps) == 0 and c.hashtable is None and c.neighbor_indices == {}


def test_make_ntuple():
    assert make_ntuple(3, 4) == (3, 3, 3, 3)
    assert make_ntuple((1, 2, 3, 4, 5), 4) == (1, 2, 3, 4)
    assert make_ntuple((1, 2), 3) == (1, 2, 2)
    with pytest.raises(TypeError):
        make_ntuple("x", 3)


def test_modules_init():
    conv = SparseConv3D(4, 8, kernel_size=3)
    assert conv.kernel_size == (3, 3, 3) and conv.stride == (1, 1, 1) and conv.weight.shape == (27, 4, 8)
    assert conv.bias is not None and SparseConv3D(4, 8, 3, bias=False).bias is None
    c2 = SparseConv3D(4, 8, kernel_size=3, stride=2, padding=1)
    assert c2.stride == (2, 2, 2) and c2.padding == (1, 1, 1)
    assert SubMConv3D(4, 8, 3).subm is True and SubMConv3D(4, 8, 5).padding == (0, 0, 0)
    assert SparseConvTransposed3D(4, 8, 3).transposed is True
    bound = 1.0 / (4 * 27) ** 0.5
    assert conv.weight.abs().max().item() <= bound
    w = conv.weight.data.clone()
    conv.reset_parameters()
    assert not torch.allclose(conv.weight.data, w)


def test_conv_requires_gpu_features():
    # The HIP kernels are the only implementation: CPU tensors are rejected loudly.
    sp = randn((16, 16, 16), batch_size=2, nnz=10, channels=4)
    conv = SubMConv3D(4, 8, 3)
    with pytest.raises(RuntimeError, match="must live on the GPU"):
        conv(sp)


def test_spatial_argument_errors():
    # tests/test_nn_functional.py:53-56 and tests/test_pooling.py:53-55 (CPU, before any kernel)
    from sparsetriton_amd.nn import SparsePooling
    from sparsetriton_amd.nn.functional import sparse_pooling

    sp = randn((16, 16, 16), batch_size=2, nnz=10, channels=4, device="cpu")
    with pytest.raises(ValueError, match="Unsupported mode"):
        sparse_pooling(sp, kernel_size=2, padding=0, stride=2, mode="invalid")
    with pytest.raises(ValueError, match="mode must be"):
        SparsePooling(kernel_size=2, mode="invalid")
