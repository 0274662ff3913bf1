"""The reference's own import lines resolve (reference tests/test_sparse_conv.py:4-5,
tests/test_utils_hash.py:3, tests/test_nn_modules.py, tests/test_config.py) and name the
implementation's objects -- one module, class and config state per name pair."""

import pytest
import torch


def test_reference_import_lines_resolve_to_the_implementation():
    from sparsetriton import SparseTensor, randn
    from sparsetriton.config import ConvAlgo, set_conv_algo
    from sparsetriton.nn.functional import sparse_conv3d
    from sparsetriton.nn.modules import SparseConv3D, SubMConv3D
    from sparsetriton.utils.hash import HashTable, flatten_coord, hash_coords, unflatten_coord

    import sparsetriton
    import sparsetriton_amd
    import sparsetriton_amd.utils.hash as impl_hash

    assert SparseTensor is sparsetriton_amd.SparseTensor and randn is sparsetriton_amd.randn
    assert HashTable is impl_hash.HashTable and flatten_coord is impl_hash.flatten_coord
    assert sparsetriton.nn is sparsetriton_amd.nn and sparsetriton.config is sparsetriton_amd.config
    assert sparse_conv3d is sparsetriton_amd.nn.functional.sparse_conv3d
    assert SubMConv3D is sparsetriton_amd.nn.SubMConv3D and SparseConv3D is sparsetriton_amd.nn.SparseConv3D
    # one config state: a setting made through either name is seen through the other
    set_conv_algo(ConvAlgo.ImplicitHashFlyGEMM)
    assert sparsetriton_amd.config.get_conv_algo() == ConvAlgo.ImplicitHashFlyGEMM
    assert callable(unflatten_coord) and callable(hash_coords)
    # the implementation modules keep their own names and specs
    assert impl_hash.__name__ == "sparsetriton_amd.utils.hash"
    assert impl_hash.__spec__.name == "sparsetriton_amd.utils.hash"


def test_reference_submodule_paths():
    import importlib

    for name in ("sparsetriton.tensor", "sparsetriton.nn.functional.conv.conv", "sparsetriton.nn.functional.conv.kmap",
                 "sparsetriton.nn.functional.conv.funcs.implicit_precomputed_gemm",
                 "sparsetriton.nn.functional.conv.funcs.implicit_hashfly_gemm", "sparsetriton.nn.functional.norm",
                 "sparsetriton.nn.functional.spatial", "sparsetriton.nn.modules.conv", "sparsetriton.nn.modules.norm",
                 "sparsetriton.nn.backbones.resnet", "sparsetriton.utils.to_dense"):
        mod = importlib.import_module(name)
        assert mod is importlib.import_module("sparsetriton_amd" + name[len("sparsetriton"):])
    with pytest.raises(ModuleNotFoundError):
        importlib.import_module("sparsetriton.no_such_module")


def test_reference_hash_helpers_via_reference_names():
    """tests/test_utils_hash.py:12-32 of the reference, through the reference's names."""
    from sparsetriton.utils.hash import flatten_coord, unflatten_coord

    c = torch.tensor([[0, 1, 2, 3], [1, 100, 200, 40], [3, 0, 0, 0]], dtype=torch.int32)
    f = flatten_coord(c)
    assert f[0].item() == (1 << 32) | (2 << 16) | 3
    assert torch.equal(unflatten_coord(f).to(torch.int32), c)


@pytest.mark.gpu
def test_reference_import_lines_run_a_submanifold_layer(device):
    """SubMConv3D forward + backward written exactly as reference code would be."""
    import numpy as np

    from oracle import oracle as O
    from sparsetriton import SparseTensor, randn
    from sparsetriton.config import ConvAlgo, set_conv_algo
    from sparsetriton.nn.functional import sparse_conv3d
    from sparsetriton.nn.modules import SubMConv3D
    from sparsetriton.utils.hash import HashTable

    for algo in (ConvAlgo.PrecomputedNeighborGEMM, ConvAlgo.ImplicitHashFlyGEMM):
        set_conv_algo(algo)
        torch.manual_seed(0)
        sp = randn((16, 16, 16), batch_size=2, channels=8, nnz=900, device=device)
        conv = SubMConv3D(8, 16, 3).to(device)
        feats = sp.F.detach().requires_grad_(True)
        sp.F = feats
        out = conv(sp)
        dY = torch.randn_like(out.F)
        out.F.backward(dY)
        c = sp.C.int().cpu().numpy()
        nbr = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, (16, 16, 16))
        W = conv.weight.detach().double().cpu().numpy()
        y = O.fwd_f64(feats.detach().cpu().numpy(), W, nbr) + conv.bias.detach().double().cpu().numpy()
        gx = O.dgrad_f64(dY.cpu().numpy(), W, nbr, c.shape[0])
        rel = lambda a, b: float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))
        assert rel(out.F.detach().cpu(), y) < 2e-3 and rel(feats.grad.cpu(), gx) < 2e-3
        # same map through the functional entry point, and the table via HashTable
        out2 = sparse_conv3d(sp, conv.weight, 3, bias=conv.bias)
        assert torch.equal(out2.F, out.F)
        t = HashTable(capacity=2 * c.shape[0], device=device)
        t.insert(sp.C)
        assert torch.equal(t.query(sp.C).cpu(), torch.arange(c.shape[0], dtype=torch.int32))
