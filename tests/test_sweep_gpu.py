"""Seeded random sweep over the convolution's geometry space through the public API
(``sparse_conv3d`` + autograd, reference ``conv.py:77-232``), each case against the float64
oracle: submanifold (odd kernel), strided and transposed convolutions; kernel 1-5 (even sizes
off the submanifold path), stride 1-3, dilation 1-2, padding within the reference's bounds;
1-3 samples, boxes of 4-22 voxels a side with 1-1,500 rows, or (a quarter of the cases) up to
53 a side with up to 20,000 rows; channel counts on and off the built
MFMA widths; fp32 / bf16 / fp16; int16 / int32 / int64 coordinates; with and without bias; a
fifth of the sets with repeated coordinates and some with rows past the box on either side; both
algorithms.  Output
coordinates equal the oracle's in order; forward, input and weight gradients within the
reference's tolerances (relative Frobenius error); an empty output is empty for the oracle too."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from sparsetriton_amd import SparseTensor
from sparsetriton_amd.config import ConvAlgo, set_conv_algo
from sparsetriton_amd.nn.functional import sparse_conv3d

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 2e-3, torch.bfloat16: 2e-2, torch.float16: 1e-2}
CHANNELS = [1, 3, 8, 16, 17, 32, 48, 64, 96, 128, 130]
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _rel(got: np.ndarray, ref: np.ndarray) -> float:
    den = float(np.linalg.norm(ref))
    num = float(np.linalg.norm(got - ref))
    return num / den if den > 0 else num


def _case(seed: int):
    rng = np.random.default_rng(70_000 + seed)
    subm = bool(rng.random() < 0.4)
    tr = (not subm) and bool(rng.random() < 0.4)
    k = int(rng.choice([1, 3, 5])) if subm else int(rng.choice([1, 2, 3, 4]))
    s = 1 if subm else int(rng.choice([1, 2, 3]))
    d = int(rng.choice([1, 1, 2]))
    if subm:
        p = (k - 1) // 2 * d
    else:
        p = int(rng.integers(0, (k - 1) * d // 2 + 1))
    B = int(rng.integers(1, 4))
    big = bool(rng.random() < 0.25)  # a quarter of the cases large enough for multi-tile plans
    lo = max(4, (k - 1) * d + 2)  # every output axis non-empty
    shape = tuple(int(v) for v in rng.integers(lo, lo + (40 if big else 14), 3))
    cells = B * shape[0] * shape[1] * shape[2]
    n = int(rng.integers(1, min(20000 if big else 1500, cells) + 1))
    lin = np.sort(rng.choice(cells, n, replace=False))
    sx, sy, sz = shape
    c = np.stack([lin // (sx * sy * sz), (lin // (sy * sz)) % sx, (lin // sz) % sy, lin % sz], 1).astype(np.int32)
    dup = bool(rng.random() < 0.2) and n >= 4
    if dup:  # repeated coordinates: a later row takes an earlier row's coordinate
        m = max(1, n // 10)
        src, dst = rng.choice(n, m, replace=False), rng.choice(n, m, replace=False)
        c[dst] = c[src]
    oob = bool(rng.random() < 0.15) and n >= 4
    if oob:  # rows past the box on one axis, either side (the reference keeps them; no row finds them)
        rows = rng.choice(n, max(1, n // 20), replace=False)
        ax = int(rng.integers(1, 4))
        past = rng.integers(0, 3, rows.shape[0])
        c[rows, ax] = np.where(rng.random(rows.shape[0]) < 0.5, shape[ax - 1] + past, -1 - past)
    cin, cout = int(rng.choice(CHANNELS)), int(rng.choice(CHANNELS))
    dtype = DTYPES[int(rng.integers(0, 3))]
    cdt = [torch.int16, torch.int32, torch.int64][int(rng.integers(0, 3))]
    bias = bool(rng.random() < 0.3)
    algo = list(ConvAlgo)[int(rng.integers(0, 2))]
    return dict(subm=subm, tr=tr, k=k, s=s, d=d, p=p, B=B, shape=shape, c=c, dup=dup, cin=cin, cout=cout,
                dtype=dtype, cdt=cdt, algo=algo, oob=oob, bias=bias, rng=rng)


@pytest.mark.parametrize("seed", range(400))
def test_random_geometry_sweep(device, seed):
    cs = _case(seed)
    subm, tr, k, s, d, p, B, shape, c = (cs[x] for x in ("subm", "tr", "k", "s", "d", "p", "B", "shape", "c"))
    cin, cout, dtype, rng = cs["cin"], cs["cout"], cs["dtype"], cs["rng"]
    n = c.shape[0]
    label = {x: (str(v) if not isinstance(v, np.ndarray) else v.shape) for x, v in cs.items() if x != "rng"}
    # operands quantised to the compute dtype so the oracle sees the same values
    X = torch.as_tensor(rng.standard_normal((n, cin)).astype(np.float32)).to(dtype).float().numpy()
    W = torch.as_tensor((rng.standard_normal((k ** 3, cin, cout)) / np.sqrt(cin * k ** 3)).astype(np.float32)).to(
        dtype).float().numpy()
    set_conv_algo(cs["algo"])
    try:
        feats = torch.as_tensor(X, device=device).to(dtype).requires_grad_(True)
        w = torch.as_tensor(W, device=device).to(dtype).requires_grad_(True)
        bvec = None
        if cs["bias"]:
            bq = torch.as_tensor(rng.standard_normal(cout).astype(np.float32)).to(dtype).float().numpy()
            bvec = torch.as_tensor(bq, device=device).to(dtype).requires_grad_(True)
        sp = SparseTensor(feats, torch.as_tensor(c, device=device).to(cs["cdt"]), spatial_shape=shape, batch_size=B)
        out = sparse_conv3d(sp, w, k, bias=bvec, stride=s, padding=p, dilation=d, transposed=tr, submanifold=subm)
        oc = out.C.cpu().numpy().astype(np.int32)
        dY = torch.as_tensor(rng.standard_normal((oc.shape[0], cout)).astype(np.float32)).to(dtype).float().numpy()
        if oc.shape[0] == 0:
            # as the reference (conv.py:161-167): an empty output is a fresh empty tensor, outside
            # the autograd graph
            assert tuple(out.F.shape) == (0, cout) and not out.F.requires_grad, label
            assert O.out_coords(c, O.target_offsets(k, d, p, tr), s, tr,
                                O.out_shape(shape, k, s, d, p, tr)).shape[0] == 0, label
            return
        out.F.backward(torch.as_tensor(dY, device=device).to(dtype))
    finally:
        set_conv_algo(ConvAlgo.PrecomputedNeighborGEMM)
    off = O.target_offsets(k, d, p, tr)
    if subm:
        assert np.array_equal(oc, c), label
        nbr = O.exact_kmap(c, c, off, 1, shape)
    else:
        new_shape = O.out_shape(shape, k, s, d, p, tr)
        assert tuple(int(v) for v in out.spatial_shape) == tuple(new_shape), label
        assert np.array_equal(oc, O.out_coords(c, off, s, tr, new_shape)), label
        if tr:
            nbr = O.exact_kmap(c, oc, off, 1, tuple(v * s for v in shape), in_scale=s)
        else:
            nbr = O.exact_kmap(c, oc, off, s, shape)
    y = O.fwd_f64_blas(X, W, nbr)
    if bvec is not None:
        y = y + bq[None, :].astype(np.float64)
        assert _rel(bvec.grad.float().cpu().numpy(), dY.astype(np.float64).sum(0)) < TOL[dtype], label
    gx = O.dgrad_f64_blas(dY, W, nbr, n)
    gw = O.wgrad_f64_blas(X, dY, nbr, k ** 3)
    tol = TOL[dtype]
    assert out.F.dtype == dtype, label
    assert _rel(out.F.detach().float().cpu().numpy(), y) < tol, label
    assert _rel(feats.grad.float().cpu().numpy(), gx) < tol, label
    assert _rel(w.grad.float().cpu().numpy(), gw) < tol, label
