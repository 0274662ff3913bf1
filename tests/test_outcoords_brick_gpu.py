"""Strided / transposed output coordinates and maps through brick indexes
(``st_outcoords_brick_*`` over the candidates' output box, ``st_kmap_strided_query``
over the input coordinates' index) against the exact oracle and against the hash-table
build, bit for bit: the output rows in first-occurrence order, the map in both
directions and the row masks.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from sparsetriton_amd import SparseTensor, workloads
from sparsetriton_amd.nn.functional import sparse_conv3d
from sparsetriton_amd.nn.functional.conv.conv import _input_table
from sparsetriton_amd.nn.functional.conv.kmap import brick_out_coords_and_map, build_out_coords_and_map

pytestmark = pytest.mark.gpu

GEOMS = [
    # k, s, p, d, transposed
    (3, 2, 1, 1, False),
    (3, 2, 0, 1, False),  # offsets 0..2: the query's general lookup path
    (5, 2, 2, 1, False),
    (3, 2, 1, 2, False),
    (3, 1, 0, 1, False),
    (3, 3, 1, 1, False),
    (2, 2, 0, 1, False),
    (3, 2, 1, 1, True),
    (3, 1, 1, 1, True),
    (3, 4, 1, 1, True),
    (5, 1, 2, 1, True),
    (2, 2, 0, 1, True),
    (3, 3, 1, 1, True),  # a stride that is not a power of two: the query's division path
    (3, 2, 2, 2, True),  # dilated offsets (-2, 0, 2) against stride 2
    (4, 3, 1, 1, True),
]


def _rand_coords(rng, n, S, B=2):
    lin = np.sort(rng.choice(B * S ** 3, n, replace=False))
    return np.stack([lin // S ** 3, (lin // S ** 2) % S, (lin // S) % S, lin % S], 1).astype(np.int32)


def _hash(device, c, shape, k, s, p, d, tr, dtype=None, chunk=None):
    """The hash-table build; coordinates of `dtype` (default: the tensor's coordinate dtype)."""
    sp = SparseTensor(torch.zeros((c.shape[0], 1), device=device), torch.as_tensor(c, device=device),
                      spatial_shape=shape)
    table = _input_table(sp, s if (tr and s > 1) else 1)
    coords = sp.C if dtype is None else torch.as_tensor(c, dtype=dtype, device=device)
    return build_out_coords_and_map(coords, shape, k, s, d, p, tr, in_table=table, with_map=True, chunk_size=chunk)


def _brick(device, c, shape, k, s, p, d, tr, dtype=None, batch_size=None, chunk=None, with_map=True):
    """The brick build; coordinates of `dtype` (default: the tensor's coordinate dtype, as conv.py
    passes them)."""
    sp = SparseTensor(torch.zeros((c.shape[0], 1), device=device), torch.as_tensor(c, device=device),
                      spatial_shape=shape)
    coords = sp.C if dtype is None else torch.as_tensor(c, dtype=dtype, device=device)
    bs = batch_size if batch_size is not None else int(c[:, 0].max()) + 1
    return brick_out_coords_and_map(coords, bs, shape, k, s, d, p, tr, with_map=with_map, chunk_size=chunk)


def _oracle(c, shape, k, s, p, d, tr, chunk=None):
    off = O.target_offsets(k, d, p, tr)
    ns = O.out_shape(shape, k, s, d, p, tr)
    oc = O.out_coords(c, off, s, tr, ns) if chunk is None else O.bf_out_coords(c, off, s, tr, ns, chunk=chunk)
    if tr:
        nbr = O.exact_kmap(c, oc, off, 1, tuple(v * s for v in shape), in_scale=s)
    else:
        nbr = O.exact_kmap(c, oc, off, s, shape)
    return oc, ns, nbr


def _same(b, h):
    """Brick build == hash build: coordinates in order, the map both ways, masks."""
    oc_b, ns_b, off_b, km_b, _ = b
    oc_h, ns_h, off_h, km_h, _ = h
    assert tuple(ns_b) == tuple(ns_h)
    assert oc_b.dtype == oc_h.dtype and torch.equal(oc_b, oc_h)
    assert torch.equal(off_b, off_h)
    assert torch.equal(km_b.nbr, km_h.nbr)
    assert torch.equal(km_b.invnbr, km_h.invnbr)
    assert torch.equal(km_b.out_masks, km_h.out_masks)
    assert torch.equal(km_b.in_masks, km_h.in_masks)


@pytest.mark.parametrize("k,s,p,d,tr", GEOMS)
def test_brick_build_exact(device, k, s, p, d, tr):
    rng = np.random.default_rng(100 * k + 10 * s + p + d + tr + 7)
    shape = (20, 20, 20)
    c = _rand_coords(rng, 1500, 20)
    b = _brick(device, c, shape, k, s, p, d, tr)
    assert b is not None
    oc, ns, nbr = _oracle(c, shape, k, s, p, d, tr)
    assert tuple(b[1]) == ns
    assert (b[0].cpu().numpy() == oc).all()
    assert (b[3].neighbor_indices.cpu().numpy() == nbr).all()
    _same(b, _hash(device, c, shape, k, s, p, d, tr))


@pytest.mark.parametrize("dtype", [torch.int16, torch.int32, torch.int64])
@pytest.mark.parametrize("tr", [False, True])
def test_brick_build_rows_outside_shape_negative_and_repeated(device, dtype, tr):
    """Rows outside [0, shape) (some negative) still yield candidates but never enter the map; a
    repeated coordinate enters it through its lowest row only (as the input hash table resolves it)."""
    rng = np.random.default_rng(31 + tr)
    c = _rand_coords(rng, 900, 14)
    c[:, 1:] -= 2  # coordinates in [-2, 12) against a (10, 11, 12) shape
    rep = c[rng.choice(c.shape[0], 120, replace=False)]
    c = np.concatenate([c, rep], 0)  # repeats, after their first rows
    c = c[rng.permutation(c.shape[0])]
    shape = (10, 11, 12)
    inside = ((rep[:, 1:] >= 0) & (rep[:, 1:] < np.array(shape))).all(1)
    b = _brick(device, c, shape, 3, 2, 1, 1, tr, dtype=dtype)
    assert b is not None
    oc, ns, nbr = _oracle(c, shape, 3, 2, 1, 1, tr)
    assert (b[0].cpu().numpy() == oc).all()
    assert (b[3].neighbor_indices.cpu().numpy() == nbr).all()
    _same(b, _hash(device, c, shape, 3, 2, 1, 1, tr, dtype=dtype))
    assert b[4].counters()["duplicate"] == int(inside.sum())  # the input index holds in-box rows only


@pytest.mark.parametrize("tr", [False, True])
@pytest.mark.parametrize("chunk", [1, 4, 9, 26, 27, 100])
def test_brick_build_chunked_order(device, tr, chunk):
    """chunk_size orders the candidates chunk by chunk (kmap.py:270-278)."""
    rng = np.random.default_rng(chunk * 2 + tr + 50)
    S = 12
    c = _rand_coords(rng, 400, S)
    shape = (S, S, S)
    b = _brick(device, c, shape, 3, 2, 1, 1, tr, chunk=chunk)
    oc, _, nbr = _oracle(c, shape, 3, 2, 1, 1, tr, chunk=chunk)
    assert (b[0].cpu().numpy() == oc).all()
    assert (b[3].neighbor_indices.cpu().numpy() == nbr).all()
    _same(b, _hash(device, c, shape, 3, 2, 1, 1, tr, chunk=chunk))
    nomap = _brick(device, c, shape, 3, 2, 1, 1, tr, chunk=chunk, with_map=False)
    assert torch.equal(nomap[0], b[0]) and nomap[3] is None


def test_brick_build_declines_rows_beyond_the_batch_count(device):
    """A candidate whose batch index lies outside [0, batch_size) cannot be indexed: the builder
    returns None (the caller then uses the hash build), never a partial result."""
    rng = np.random.default_rng(5)
    c = _rand_coords(rng, 300, 10, B=3)
    assert _brick(device, c, (10, 10, 10), 3, 2, 1, 1, False, batch_size=2) is None
    assert _brick(device, c, (10, 10, 10), 3, 2, 1, 1, False, batch_size=3) is not None
    # rows of a batch beyond the count whose candidates are all filtered out do not matter
    one = np.array([[0, 2, 2, 2], [5, 1, 1, 1]], np.int32)  # stride 2, padding 0: (1,1,1) has no output
    b = _brick(device, one, (8, 8, 8), 1, 2, 0, 1, False, batch_size=1)
    assert b is not None and b[0].cpu().numpy().tolist() == [[0, 1, 1, 1]]


def test_brick_build_all_filtered(device):
    b = _brick(device, np.array([[0, 1, 1, 1]], np.int32), (2, 2, 2), 1, 2, 0, 1, False)
    assert b is not None and b[0].shape == (0, 4)
    assert b[3].nbr.shape == (1, 0)


@pytest.fixture(scope="module")
def cfg2():
    return workloads.config2()


def test_config3_config4_brick_builds_exact(device, cfg2):
    c, shape = cfg2
    b3 = _brick(device, c, shape, 3, 2, 1, 1, False)
    oc3, ns3, nbr3 = _oracle(c, shape, 3, 2, 1, 1, False)
    assert tuple(b3[1]) == ns3 == (720, 720, 21)
    assert (b3[0].cpu().numpy() == oc3).all()
    assert (b3[3].neighbor_indices.cpu().numpy() == nbr3).all()
    _same(b3, _hash(device, c, shape, 3, 2, 1, 1, False))
    b4 = _brick(device, oc3, ns3, 3, 2, 1, 1, True)
    oc4, ns4, nbr4 = _oracle(oc3, ns3, 3, 2, 1, 1, True)
    assert tuple(b4[1]) == ns4 == (1439, 1439, 41)
    assert (b4[0].cpu().numpy() == oc4).all()
    assert (b4[3].neighbor_indices.cpu().numpy() == nbr4).all()
    _same(b4, _hash(device, oc3, ns3, 3, 2, 1, 1, True))


@pytest.mark.parametrize("tr", [False, True])
def test_conv_uses_the_brick_build(device, tr):
    """sparse_conv3d's strided / transposed precomputed path builds through the brick indexes
    (no input hash table is made) and matches the float64 oracle."""
    rng = np.random.default_rng(77 + tr)
    S, n, cin, cout = 12, 700, 8, 12
    c = _rand_coords(rng, n, S)
    X = rng.standard_normal((n, cin)).astype(np.float32)
    W = (rng.standard_normal((27, cin, cout)) / np.sqrt(27 * cin)).astype(np.float32)
    sp = SparseTensor(torch.as_tensor(X, device=device), torch.as_tensor(c, device=device), spatial_shape=(S,) * 3)
    out = sparse_conv3d(sp, torch.as_tensor(W, device=device), 3, stride=2, padding=1, transposed=tr,
                        submanifold=False)
    assert sp._cache.hashtable is None and not any(isinstance(k, tuple) and k[0] == "scaled_table"
                                                   for k in sp._cache.kmaps)
    oc, _, nbr = _oracle(c, (S,) * 3, 3, 2, 1, 1, tr)
    assert (out.C.cpu().numpy() == oc).all()
    ref = O.fwd_f64(X.astype(np.float64), W.astype(np.float64), nbr)
    got = out.F.detach().cpu().numpy().astype(np.float64)
    assert np.abs(got - ref).max() <= 2e-3 * max(np.abs(ref).max(), 1.0)


@pytest.mark.parametrize("S", [32, 256])
def test_brick_plan_flags_offsets_beyond_the_kernel_bound(device, S):
    """A C-ABI caller whose offsets reach more outputs than kernel_size / dilation bound (here
    the 27 offsets of a 3x3x3 kernel declared as kernel_size 1, so the output index is sized for
    one output per input): the plan counts ST_STATUS_OVERFLOW, reports no outputs and writes no
    level-2 word or rank past the index's bound; emit writes nothing and the inverse map is all
    -1.  At S = 32 the voxels overflow (the output box has fewer bricks than rows), at S = 256 the
    occupied bricks do.  The same call with the kernel's own size then builds the exact outputs
    (a regression test of the bounds: the guarded build must leave the workspace reusable)."""
    import ctypes

    from sparsetriton_amd import _lib
    from sparsetriton_amd.nn.functional.conv.kmap import _offsets_i32, _target_offsets, out_spatial_shape

    rng = np.random.default_rng(5)
    n = 2000
    c = _rand_coords(rng, n, S)
    coords = torch.as_tensor(c, device=device)
    shape = (S, S, S)
    k, s, p, d = 3, 2, 1, 1
    offs = _offsets_i32(_target_offsets(k, d, p, False, device))
    ns = out_spatial_shape(shape, k, s, d, p, False)
    g = _lib.OutGeom()
    g.K, g.transposed, g.stride, g.chunk = offs.shape[0], 0, s, 0
    for a in range(3):
        g.in_shape[a], g.out_shape[a] = shape[a], ns[a]
    lib = _lib.lib()
    st = _lib.stream_of(device)

    def plan(kernel_size):
        wb, nb = ctypes.c_int64(), ctypes.c_int64()
        assert lib.st_outcoords_brick_sizes(n, ctypes.byref(g), 2, kernel_size, d, ctypes.byref(wb),
                                            ctypes.byref(nb)) == 0
        work = torch.full((wb.value,), 0xAB, dtype=torch.uint8, device=device)
        counts = torch.empty((nb.value + 1,), dtype=torch.int32, device=device)
        status = torch.empty((_lib.STATUS_WORDS,), dtype=torch.int32, device=device)
        _lib.call("st_outcoords_brick_plan", _lib.ptr(coords), _lib.coord_code(coords.dtype), n, _lib.ptr(offs),
                  ctypes.byref(g), 2, kernel_size, d, _lib.ptr(work), wb.value, _lib.ptr(counts), nb.value,
                  _lib.ptr(status), st)
        return work, wb.value, counts, nb.value, status

    work, wb, counts, nb, status = plan(1)
    assert int(status[_lib.STATUS_OVERFLOW]) > 0
    assert int(counts[nb]) == 0
    out = torch.full((4, 4), -7, dtype=coords.dtype, device=device)
    _lib.call("st_outcoords_brick_emit", _lib.ptr(coords), _lib.coord_code(coords.dtype), n, _lib.ptr(offs),
              ctypes.byref(g), 2, 1, d, _lib.ptr(work), wb, _lib.ptr(counts), nb, _lib.ptr(out), 4, st)
    assert bool((out == -7).all())
    from sparsetriton_amd.nn.functional.conv.kmap import BrickIndex

    index = BrickIndex.build(coords, 2, shape)
    K, W = offs.shape[0], 1
    inv = torch.full((K, n), 5, dtype=torch.int32, device=device)
    masks = torch.full((n, W), 5, dtype=torch.int32, device=device)
    _lib.call("st_outcoords_brick_inverse", _lib.ptr(coords), _lib.coord_code(coords.dtype), n, _lib.ptr(offs),
              ctypes.byref(g), 2, 1, d, _lib.ptr(work), wb, _lib.ptr(index.work), index.nbytes, _lib.ptr(inv),
              _lib.ptr(masks), st)
    assert bool((inv == -1).all()) and bool((masks == 0).all())

    _, _, counts3, nb3, status3 = plan(k)
    assert int(status3[_lib.STATUS_OVERFLOW]) == 0
    oc = O.out_coords(c, O.target_offsets(k, d, p, False), s, False, O.out_shape(shape, k, s, d, p, False))
    assert int(counts3[nb3]) == oc.shape[0]
    b = _brick(device, c, shape, k, s, p, d, False, batch_size=2)
    assert b is not None and np.array_equal(b[0].cpu().numpy(), oc)
