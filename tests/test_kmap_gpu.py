"""Kernel maps and output coordinates on the GPU vs the exact oracle (bit-exact).

Submanifold maps are compared entry by entry; strided / transposed output
coordinates are compared in order (first occurrence in the input-major /
offset-minor candidate enumeration) and their maps entry by entry, which
implies equality of the canonical sorted (in, out, k) triples.  The
transposed map is checked for consistency with the forward map, and the row
masks against the map.  Full-size benchmark coordinate sets are included.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from sparsetriton_amd import SparseTensor, workloads
from sparsetriton_amd.nn.functional import sparse_conv3d
from sparsetriton_amd.nn.functional.conv.conv import _input_table, compute_neighbor_indices
from sparsetriton_amd.nn.functional.conv.kmap import (
    _target_offsets,
    brick_out_coords_and_map,
    build_out_coords,
    build_out_coords_and_map,
    query_kernel_map,
)

pytestmark = pytest.mark.gpu


def _rand_coords(rng, n, S, B=2):
    lin = np.sort(rng.choice(B * S ** 3, n, replace=False))
    return np.stack([lin // S ** 3, (lin // S ** 2) % S, (lin // S) % S, lin % S], 1).astype(np.int32)


def _check_masks(kmap):
    nbr = kmap.neighbor_indices.cpu().numpy().T  # (K, N)
    K = kmap.K
    bits = (nbr >= 0).astype(np.uint64)
    expect = np.zeros((kmap.n_out,), dtype=np.uint64)
    for k in range(min(K, 32)):
        expect |= bits[k] << np.uint64(k)
    got = kmap.out_masks.cpu().numpy()[:, 0].astype(np.uint32).astype(np.uint64)
    assert (got == expect).all()


def _check_inverse(kmap):
    kmap.ensure_inverse()
    nbr = kmap.neighbor_indices.cpu().numpy().T  # (K, N_out)
    inv = kmap.invnbr.cpu().numpy()  # (K, N_in)
    K = kmap.K
    for k in range(K):
        o = np.nonzero(nbr[k] >= 0)[0]
        assert (inv[k, nbr[k, o]] == o).all()
        assert (inv[k] >= 0).sum() == o.shape[0]
    in_bits = (inv >= 0)
    got = kmap.in_masks.cpu().numpy()[:, 0].astype(np.uint32)
    expect = np.zeros(kmap.n_in, dtype=np.uint64)
    for k in range(min(K, 32)):
        expect |= in_bits[k].astype(np.uint64) << np.uint64(k)
    assert (got.astype(np.uint64) == expect).all()


def _subm(device, c, shape, k=3, d=1, dtype=torch.int16):
    coords = torch.as_tensor(c, dtype=dtype, device=device)
    sp = SparseTensor(torch.zeros((c.shape[0], 1), device=device), coords, spatial_shape=shape)
    table = _input_table(sp, 1)
    offs = _target_offsets(k, d, (k - 1) * d // 2, False, device)
    return query_kernel_map(table, sp.C, offs, shape, 1, c.shape[0])


@pytest.mark.parametrize("k,d", [(3, 1), (5, 1), (3, 2)])
def test_subm_kmap_exact(device, k, d):
    rng = np.random.default_rng(k + d)
    c = _rand_coords(rng, 3000, 24)
    kmap = _subm(device, c, (24, 24, 24), k, d)
    off = O.target_offsets(k, d, (k - 1) * d // 2, False)
    expect = O.exact_kmap(c, c, off, 1, (24, 24, 24))
    assert (kmap.neighbor_indices.cpu().numpy() == expect).all()
    if k ** 3 <= 32:
        _check_masks(kmap)
        _check_inverse(kmap)


def test_subm_kmap_out_of_bounds_rows(device):
    rng = np.random.default_rng(5)
    c = _rand_coords(rng, 2000, 20)
    shape = (15, 18, 20)  # some coordinates lie outside: their neighbours are dropped, as in conv.py:55-59
    kmap = _subm(device, c, shape)
    expect = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, shape)
    assert (kmap.neighbor_indices.cpu().numpy() == expect).all()
    _check_inverse(kmap)


def test_compute_neighbor_indices_api(device):
    rng = np.random.default_rng(6)
    c = _rand_coords(rng, 1000, 16)
    coords = torch.as_tensor(c, dtype=torch.int32, device=device)
    sp = SparseTensor(torch.zeros((1000, 1), device=device), coords, spatial_shape=(16, 16, 16))
    table = _input_table(sp, 1)
    offs = _target_offsets(3, 1, 1, False, device).to(sp.C.dtype)
    nbr = compute_neighbor_indices(table, sp.C, offs, (16, 16, 16), 1)
    assert nbr.shape == (1000, 27) and nbr.dtype == torch.int32
    assert (nbr.cpu().numpy() == O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, (16, 16, 16))).all()


GEOMS = [
    # k, s, p, d, transposed
    (3, 2, 1, 1, False),
    (5, 2, 2, 1, False),
    (3, 2, 1, 2, False),
    (3, 1, 0, 1, False),
    (3, 3, 1, 1, False),
    (3, 2, 1, 1, True),
    (3, 1, 1, 1, True),
    (3, 4, 1, 1, True),
    (5, 1, 2, 1, True),
]


def _strided(device, c, shape, k, s, p, d, tr, dtype=torch.int16):
    coords = torch.as_tensor(c, dtype=dtype, device=device)
    sp = SparseTensor(torch.zeros((c.shape[0], 1), device=device), coords, spatial_shape=shape)
    scale = s if (tr and s > 1) else 1
    table = _input_table(sp, scale)
    return build_out_coords_and_map(sp.C, shape, k, s, d, p, tr, in_table=table, with_map=True)


def _oracle_strided(c, shape, k, s, p, d, tr):
    off = O.target_offsets(k, d, p, tr)
    ns = O.out_shape(shape, k, s, d, p, tr)
    oc = O.out_coords(c, off, s, tr, ns)
    if tr:
        nbr = O.exact_kmap(c, oc, off, 1, tuple(v * s for v in shape), in_scale=s)
    else:
        nbr = O.exact_kmap(c, oc, off, s, shape)
    return oc, ns, nbr


@pytest.mark.parametrize("k,s,p,d,tr", GEOMS)
def test_strided_transposed_exact(device, k, s, p, d, tr):
    rng = np.random.default_rng(100 * k + 10 * s + p + d + tr)
    shape = (20, 20, 20)
    c = _rand_coords(rng, 1500, 20)
    out_coords, ns, offsets, kmap, _ = _strided(device, c, shape, k, s, p, d, tr)
    oc, ns_o, nbr = _oracle_strided(c, shape, k, s, p, d, tr)
    assert tuple(ns) == ns_o
    assert out_coords.dtype == torch.int16
    assert (out_coords.cpu().numpy() == oc).all()
    assert (kmap.neighbor_indices.cpu().numpy() == nbr).all()
    assert (offsets.cpu().numpy() == O.target_offsets(k, d, p, tr)).all()
    if k ** 3 <= 32:
        _check_masks(kmap)
        inv = kmap.invnbr.clone()
        kmap.invnbr = None
        _check_inverse(kmap)  # invert kernel == map emitted with the coordinates
        assert torch.equal(kmap.invnbr, inv)


def test_build_out_coords_api(device):
    rng = np.random.default_rng(9)
    c = torch.as_tensor(_rand_coords(rng, 500, 12), dtype=torch.int16, device=device)
    oc, ns, offs = build_out_coords(c, (12, 12, 12), 3, stride=2, padding=1, submanifold=False)
    expect = O.out_coords(c.cpu().numpy(), O.target_offsets(3, 1, 1, False), 2, False, (6, 6, 6))
    assert tuple(ns) == (6, 6, 6) and (oc.cpu().numpy() == expect).all()
    # submanifold short-circuit and the reference docstring KAT (kmap.py:477-484)
    one = torch.tensor([[0, 1, 1, 1]], dtype=torch.int16, device=device)
    oc1, ns1, _ = build_out_coords(one, (8, 8, 8), 3, stride=1, padding=1)
    assert oc1 is one and oc1.shape[1] == 4


@pytest.mark.parametrize("tr", [False, True])
@pytest.mark.parametrize("chunk", [1, 4, 9, 26, 27, 100])
def test_chunked_out_coords(device, tr, chunk):
    """chunk_size orders the candidates chunk by chunk (kmap.py:270-278) and sizes the dedup table by the
    distinct outputs (small chunks start with a table too small for them, which must grow)."""
    rng = np.random.default_rng(chunk * 2 + tr)
    S = 12
    c = _rand_coords(rng, 400, S)
    shape = (S, S, S)
    off = O.target_offsets(3, 1, 1, tr)
    ns = O.out_shape(shape, 3, 2, 1, 1, tr)
    expect = O.bf_out_coords(c, off, 2, tr, ns, chunk=chunk)
    ct = torch.as_tensor(c, dtype=torch.int16, device=device)
    oc, ns_gpu, _ = build_out_coords(ct, shape, 3, stride=2, padding=1, transposed=tr, submanifold=False,
                                     chunk_size=chunk)
    assert tuple(ns_gpu) == tuple(ns)
    assert (oc.cpu().numpy() == expect).all()
    sp = SparseTensor(torch.zeros((c.shape[0], 1), device=device), ct, spatial_shape=shape)
    table = _input_table(sp, 2 if tr else 1)
    oc2, _, _, kmap, _ = build_out_coords_and_map(sp.C, shape, 3, 2, 1, 1, tr, in_table=table, with_map=True,
                                                  chunk_size=chunk)
    assert torch.equal(oc2, oc)
    if tr:
        nbr = O.exact_kmap(c, oc2.cpu().numpy(), off, 1, tuple(v * 2 for v in shape), in_scale=2)
    else:
        nbr = O.exact_kmap(c, oc2.cpu().numpy(), off, 2, shape)
    assert (kmap.neighbor_indices.cpu().numpy() == nbr).all()


def test_duplicate_inputs_use_table_row(device):
    c = np.array([[0, 2, 2, 2], [0, 3, 2, 2], [0, 2, 2, 2], [0, 5, 5, 5]], dtype=np.int32)
    out_coords, ns, _, kmap, _ = _strided(device, c, (8, 8, 8), 3, 2, 1, 1, False)
    oc, _, nbr = _oracle_strided(c, (8, 8, 8), 3, 2, 1, 1, False)  # oracle keeps the lowest row per coordinate
    assert (out_coords.cpu().numpy() == oc).all()
    assert (kmap.neighbor_indices.cpu().numpy() == nbr).all()


def test_empty_and_all_filtered(device):
    e = np.zeros((0, 4), dtype=np.int32)
    out_coords, ns, _, kmap, _ = _strided(device, e, (8, 8, 8), 3, 2, 1, 1, False)
    assert out_coords.shape == (0, 4)
    # stride 2, padding 0: a single voxel at an odd coordinate has no even-aligned output
    out_coords, _, _, _, _ = _strided(device, np.array([[0, 1, 1, 1]], np.int32), (2, 2, 2), 1, 2, 0, 1, False)
    assert out_coords.shape == (0, 4)


# ------------------------------------------------------------ benchmark sizes

@pytest.fixture(scope="module")
def cfg2():
    return workloads.config2()


def test_config2_subm_kmap_exact(device, cfg2):
    c, shape = cfg2
    kmap = _subm(device, c, shape)
    expect = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, shape)
    got = kmap.neighbor_indices.cpu().numpy()
    assert (got == expect).all()
    _check_masks(kmap)
    p = int((expect >= 0).sum())
    assert 3 * c.shape[0] <= p <= 8 * c.shape[0]


def test_config3_config4_maps_exact(device, cfg2):
    c, shape = cfg2
    out3, ns3, _, kmap3, _ = _strided(device, c, shape, 3, 2, 1, 1, False)
    oc3, ns3o, nbr3 = _oracle_strided(c, shape, 3, 2, 1, 1, False)
    assert tuple(ns3) == ns3o == (720, 720, 21)
    assert (out3.cpu().numpy() == oc3).all()
    assert (kmap3.neighbor_indices.cpu().numpy() == nbr3).all()
    # transposed k3 s2 p1 on the strided output (config 4)
    out4, ns4, _, kmap4, _ = _strided(device, oc3, ns3o, 3, 2, 1, 1, True)
    oc4, ns4o, nbr4 = _oracle_strided(oc3, ns3o, 3, 2, 1, 1, True)
    assert tuple(ns4) == ns4o == (1439, 1439, 41)
    assert (out4.cpu().numpy() == oc4).all()
    assert (kmap4.neighbor_indices.cpu().numpy() == nbr4).all()


# ------------------------------------------------- tile plans and pair lists

def test_tile_plan_and_pair_list(device):
    rng = np.random.default_rng(31)
    c = _rand_coords(rng, 5000, 24)
    kmap = _subm(device, c, (24, 24, 24))
    nbr = kmap.neighbor_indices.cpu().numpy().T  # (K, N)
    K, N = nbr.shape
    assert kmap.nbr.is_contiguous() and kmap.nbr.shape == (K, N)
    for plan, masks in ((kmap.forward_plan(), kmap.out_masks), (kmap.backward_plan(), None)):
        if masks is None:
            masks = kmap.in_masks
        perm = plan.perm.cpu().numpy()
        assert np.array_equal(np.sort(perm), np.arange(N))
        sorted_keys = _fold_keys(masks.cpu().numpy().view(np.uint32), K)[perm]
        assert (np.diff(sorted_keys.astype(np.int64)) >= 0).all()  # stable radix order by mask key
        # stability: equal keys keep ascending row order
        same = sorted_keys[1:] == sorted_keys[:-1]
        assert (perm[1:][same] > perm[:-1][same]).all()
    # tile plan: each 128-row tile (perm order) lists the union of its rows' offsets and,
    # per listed offset, the map entries of its rows contiguously
    tiles = kmap.forward_tiles()
    perm = kmap.forward_plan().perm.cpu().numpy()
    nk = tiles.nk.cpu().numpy()
    kl = tiles.klist.cpu().numpy().reshape(-1, K)
    tm = tiles.tmap.cpu().numpy().reshape(-1, K, 128)
    ntiles = (N + 127) // 128
    for t in range(ntiles):
        rows = perm[t * 128:(t + 1) * 128]
        active = np.nonzero((nbr[:, rows] >= 0).any(axis=1))[0]
        assert nk[t] == len(active) and np.array_equal(kl[t, :nk[t]], active)
        expect = np.full((len(active), 128), -1, dtype=np.int32)
        expect[:, :len(rows)] = nbr[active][:, rows]
        assert np.array_equal(tm[t, :nk[t]], expect)
    pl = kmap.pair_list(chunk=100)
    ks = pl.kstart.cpu().numpy()
    cs = pl.cstart.cpu().numpy()
    P = int(ks[-1])
    pairs = pl.pairs.cpu().numpy()[: 2 * P].reshape(-1, 2)
    expect = []
    for k in range(K):
        o = np.nonzero(nbr[k] >= 0)[0]
        expect.append(np.stack([nbr[k, o], o], 1))
        assert ks[k + 1] - ks[k] == o.shape[0]
        assert cs[k + 1] - cs[k] == (o.shape[0] + 99) // 100
    assert np.array_equal(pairs, np.concatenate(expect))
    assert cs[-1] <= pl.max_chunks
    # chunk order: the real chunks first, stably sorted by the 9-bit bucket of their first output row
    corder = pl.corder.cpu().numpy()
    total = int(cs[-1])
    assert np.array_equal(np.sort(corder), np.arange(pl.max_chunks))
    bucket = []
    for cidx in range(total):
        k = int(np.searchsorted(cs, cidx, side="right") - 1)
        p0 = ks[k] + (cidx - cs[k]) * 100
        bucket.append(pairs[p0, 1] * 512 // N)
    assert np.array_equal(corder[:total], np.argsort(np.array(bucket), kind="stable"))


def _chunk_order_ref(pairs, ks, cs, chunk, n_out, max_chunks):
    total = int(cs[-1])
    bucket = []
    for cidx in range(total):
        k = int(np.searchsorted(cs, cidx, side="right") - 1)
        p0 = ks[k] + (cidx - cs[k]) * chunk
        bucket.append(min(pairs[p0, 1] * 512 // n_out, 511))
    return np.concatenate([np.argsort(np.array(bucket, dtype=np.int64), kind="stable"), np.arange(total, max_chunks)])


@pytest.mark.parametrize("k,chunk", [(3, 2048), (3, 64), (3, 8), (5, 512)])
def test_one_call_plans_match_the_separate_builders(device, k, chunk):
    """st_kmap_plans (sort + tile plan on the caller's stream, pair list + chunk order on the
    library's side stream) gives the same buffers as the separate entry points; chunk 8 has more
    chunks, and the 5x5x5 kernel more offsets, than the one-workgroup chunk order holds (the keys +
    radix sort route)."""
    from sparsetriton_amd.nn.functional.conv.kmap import MapPlan, PairList, TileMap, TilePlan
    rng = np.random.default_rng(32)
    c = _rand_coords(rng, 5000, 24)
    kmap = _subm(device, c, (24, 24, 24), k=k)
    kmap.ensure_out_masks()
    K, N = kmap.K, kmap.n_out
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):  # a caller's non-default stream
        plan = MapPlan.build(kmap.nbr, kmap.k_stride, kmap.r_stride, kmap.out_masks, K, N, kmap.n_in, chunk)
        perm = TilePlan.build(N, K, kmap.out_masks).perm
        tiles = TileMap.build(kmap.nbr, kmap.k_stride, kmap.r_stride, kmap.out_masks, K, perm, N, kmap.n_in)
        pl = PairList.build(kmap.nbr, kmap.k_stride, kmap.r_stride, N, K, kmap.n_in, chunk)
    torch.cuda.synchronize()
    assert torch.equal(plan.tiles.perm, perm)
    assert torch.equal(plan.tiles.nk, tiles.nk)
    nt = tiles.nk.shape[0]
    kl_a, kl_b = plan.tiles.klist.view(nt, K), tiles.klist.view(nt, K)
    tm_a, tm_b = plan.tiles.tmap.view(nt, K, 128), tiles.tmap.view(nt, K, 128)
    for t in range(nt):
        n = int(tiles.nk[t])
        assert torch.equal(kl_a[t, :n], kl_b[t, :n]) and torch.equal(tm_a[t, :n], tm_b[t, :n])
    q = plan.pairs
    assert q.max_chunks == pl.max_chunks and q.chunk == pl.chunk == chunk
    assert torch.equal(q.kstart, pl.kstart) and torch.equal(q.cstart, pl.cstart)
    P = int(pl.kstart[-1])
    assert torch.equal(q.pairs[:2 * P], pl.pairs[:2 * P])
    assert torch.equal(q.corder, pl.corder[:q.max_chunks])
    ks, cs = pl.kstart.cpu().numpy(), pl.cstart.cpu().numpy()
    ref = _chunk_order_ref(pl.pairs.cpu().numpy()[:2 * P].reshape(-1, 2), ks, cs, chunk, N, pl.max_chunks)
    assert np.array_equal(q.corder.cpu().numpy(), ref)



@pytest.mark.parametrize("n,S", [(5000, 24), (300000, 64)])
def test_pair_list_chooses_its_chunk_size(device, n, S):
    """ST_PAIR_CHUNK_AUTO: the size is the least power of two >= 1024 with P <= 2048 * size,
    stored after cstart; the list, its chunk starts and its chunk order equal those built with
    that size given, through both builders; the weight gradient over either is the same."""
    from sparsetriton_amd.nn.functional.conv.kmap import MapPlan, PairList
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import wgrad
    rng = np.random.default_rng(33)
    c = _rand_coords(rng, n, S)
    kmap = _subm(device, c, (S, S, S))
    kmap.ensure_out_masks()
    K, N = kmap.K, kmap.n_out
    auto = PairList.build(kmap.nbr, kmap.k_stride, kmap.r_stride, N, K, kmap.n_in, -1)
    plan = MapPlan.build(kmap.nbr, kmap.k_stride, kmap.r_stride, kmap.out_masks, K, N, kmap.n_in, -1).pairs
    P = int((kmap.nbr >= 0).sum())
    size = 1024
    while size * 2048 < P:
        size *= 2
    assert auto.chunk_size() == plan.chunk_size() == size
    assert auto.max_chunks == plan.max_chunks == min(2048 + K, K * N // 1024 + K)
    fixed = PairList.build(kmap.nbr, kmap.k_stride, kmap.r_stride, N, K, kmap.n_in, size)
    for q in (auto, plan):
        assert torch.equal(q.kstart, fixed.kstart) and torch.equal(q.cstart, fixed.cstart)
        assert int(q.cstart[-1]) <= q.max_chunks
        assert torch.equal(q.pairs[:2 * P], fixed.pairs[:2 * P])
        total = int(fixed.cstart[-1])
        assert torch.equal(q.corder[:total], fixed.corder[:total])
        assert np.array_equal(np.sort(q.corder.cpu().numpy()), np.arange(q.max_chunks))
    X = torch.randn((N, 32), device=device)
    dY = torch.randn((N, 48), device=device)
    dw = [wgrad(X, dY, kmap, torch.float32, pairs=q) for q in (auto, plan, fixed)]
    assert torch.equal(dw[0], dw[2]) and torch.equal(dw[1], dw[2])

@pytest.mark.parametrize("n", [4096, 6000, 9001, 12288])
def test_pair_list_wide_loads_equal_the_scalar_pass(device, n):
    """A map with contiguous rows and 16-byte aligned columns takes the 16-byte-load count / emit
    kernels; the same map with a padded column stride takes the 4-byte ones: identical lists
    (pairs sorted by (offset, output row)), also across partial last row blocks."""
    from sparsetriton_amd.nn.functional.conv.kmap import PairList
    rng = np.random.default_rng(n)
    K = 27
    n_in = 5000
    nbr = torch.as_tensor(rng.integers(-3 * n_in, n_in, size=(K, n)), dtype=torch.int32, device=device)
    nbr[nbr < 0] = -1
    nbr[3, ::7] = n_in + 5  # out-of-range sources are not pairs
    padded = torch.full((K, n + 3), -1, dtype=torch.int32, device=device)
    padded[:, :n] = nbr
    for chunk in (-1, 1024):
        a = PairList.build(nbr, n, 1, n, K, n_in, chunk)              # 16-byte loads when n % 4 == 0
        b = PairList.build(padded, n + 3, 1, n, K, n_in, chunk)       # 4-byte loads
        P = int(((nbr >= 0) & (nbr < n_in)).sum())
        assert torch.equal(a.kstart, b.kstart) and torch.equal(a.cstart, b.cstart)
        assert int(a.kstart[-1]) == P
        assert torch.equal(a.pairs[:2 * P], b.pairs[:2 * P])
        got = a.pairs[:2 * P].view(-1, 2).cpu().numpy()
        ks, os_ = np.nonzero(((nbr >= 0) & (nbr < n_in)).cpu().numpy())
        assert (got[:, 1] == os_).all() and (got[:, 0] == nbr.cpu().numpy()[ks, os_]).all()


def test_one_call_plans_of_an_empty_map(device):
    from sparsetriton_amd.nn.functional.conv.kmap import MapPlan
    nbr = torch.empty((27, 0), dtype=torch.int32, device=device)
    masks = torch.empty((0, 1), dtype=torch.int32, device=device)
    plan = MapPlan.build(nbr, 0, 1, masks, 27, 0, 0, 2048)
    torch.cuda.synchronize()
    assert plan.pairs.kstart.cpu().tolist() == [0] * 28 and plan.pairs.cstart.cpu().tolist() == [0] * 28
    assert plan.pairs.corder.cpu().tolist() == list(range(27))


@pytest.mark.parametrize("k,d", [(3, 1), (5, 1), (3, 2)])
def test_subm_map_is_its_own_transpose(device, k, d):
    """An odd-kernel submanifold map read with offsets reversed equals the explicit
    transposed map (st_kmap_invert), which the symmetric input gradient relies on."""
    rng = np.random.default_rng(40 + k + d)
    c = _rand_coords(rng, 7000, 20)
    kmap = _subm(device, c, (20, 20, 20), k=k, d=d)
    kmap.ensure_inverse()
    assert torch.equal(kmap.invnbr, kmap.nbr.flip(0))
    K = k ** 3
    bits = np.unpackbits(kmap.out_masks.cpu().numpy().view(np.uint8), axis=1, bitorder="little")[:, :K]
    ibits = np.unpackbits(kmap.in_masks.cpu().numpy().view(np.uint8), axis=1, bitorder="little")[:, :K]
    assert np.array_equal(ibits, bits[:, ::-1])
    # input gradient through the symmetric map == through the explicit transpose
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import gather_gemm_dgrad
    from sparsetriton_amd.nn.functional.conv.kmap import KernelMap
    explicit = KernelMap(kmap.nbr, kmap.n_in, kmap.n_out, K, out_masks=kmap.out_masks, invnbr=kmap.invnbr,
                         in_masks=kmap.in_masks)
    sym = KernelMap(kmap.nbr, kmap.n_in, kmap.n_out, K, out_masks=kmap.out_masks, symmetric=True)
    for dtype, tol in ((torch.float32, 1e-5), (torch.bfloat16, 1e-2)):
        dY = torch.randn(kmap.n_out, 48, device=device, dtype=dtype)
        W = torch.randn(K, 40, 48, device=device, dtype=dtype)
        a = gather_gemm_dgrad(dY, sym, W).float()
        b = gather_gemm_dgrad(dY, explicit, W).float()
        assert (torch.linalg.norm(a - b) / torch.linalg.norm(b)).item() < tol


def _fold_keys(masks, K):
    """32-bit sort key of a (n, W) mask array: word w rotated left by 7w, xor-folded; for K = 27
    the bits then reordered: offsets ranked by the number of axes (0..3) on which
    (k // 9, k // 3 % 3, k % 3) differs from the centre (1, 1, 1), ties by index."""
    m = masks.astype(np.uint64)
    key = m[:, 0].copy()
    for w in range(1, m.shape[1]):
        r = (7 * w) & 31
        key ^= ((m[:, w] << np.uint64(r)) | (m[:, w] >> np.uint64(32 - r))) & np.uint64(0xFFFFFFFF) if r else m[:, w]
    if K == 27:
        axes = [sum(int(v != 1) for v in (k // 9, k // 3 % 3, k % 3)) for k in range(27)]
        rank = sorted(range(27), key=lambda k: (axes[k], k))
        pos = {k: p for p, k in enumerate(rank)}
        assert [pos[k] for k in (13, 4, 0, 26)] == [0, 1, 19, 26]  # centre, first face, first/last corner
        out = np.zeros_like(key)
        for k in range(27):
            out |= ((key >> np.uint64(k)) & np.uint64(1)) << np.uint64(pos[k])
        key = out
    return key.astype(np.uint32)


@pytest.mark.parametrize("n,K", [(0, 27), (1, 27), (1025, 27), (4095, 8), (4097, 1), (300_001, 27), (123_457, 125),
                                 (70_000, 343), (1_100_000, 27), (4_500_000, 27)])
def test_sort_rows_stable(device, n, K):
    """st_kmap_sort_rows is a stable sort of rows by their (folded) offset mask:
    equal to numpy's stable argsort across many tiles and all digits (1.1M rows: 1075 tiles of
    1024 rows, so the per-digit column scans take three 512-tile batches; 4.5M rows take the
    4096-row tiles of large inputs)."""
    from sparsetriton_amd.nn.functional.conv.kmap import TilePlan
    rng = np.random.default_rng(n + K)
    W = (K + 31) // 32
    # few distinct masks (long equal runs test stability) mixed with random ones
    pool = rng.integers(0, 2**32, size=(64, W), dtype=np.uint64).astype(np.uint32)
    if K % 32:
        pool[:, -1] &= np.uint32((1 << (K % 32)) - 1)
    masks = pool[rng.integers(0, 64, size=n)]
    rnd = rng.random(n) < 0.3
    masks[rnd] = rng.integers(0, 2**32, size=(int(rnd.sum()), W), dtype=np.uint64).astype(np.uint32)
    if K % 32 and n:
        masks[:, -1] &= np.uint32((1 << (K % 32)) - 1)
    m_t = torch.from_numpy(masks.view(np.int32).copy()).to(device)
    perm = TilePlan.build(n, K, m_t).perm.cpu().numpy()
    expect = np.argsort(_fold_keys(masks, K), kind="stable")
    assert np.array_equal(perm, expect)


def test_wgrad_scan_matches_pairs(device):
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import wgrad, wgrad_scan
    rng = np.random.default_rng(32)
    c = _rand_coords(rng, 6000, 24)
    kmap = _subm(device, c, (24, 24, 24))
    for dtype in (torch.float32, torch.bfloat16):
        X = torch.randn(6000, 32, device=device, dtype=dtype)
        dY = torch.randn(6000, 48, device=device, dtype=dtype)
        a = wgrad(X, dY, kmap, torch.float32)
        b = wgrad_scan(X, dY, kmap, torch.float32)
        ref = O.wgrad_f64(X.float().cpu().numpy(), dY.float().cpu().numpy(), kmap.neighbor_indices.cpu().numpy(), 27)
        for r in (a, b):
            err = np.linalg.norm(r.cpu().numpy() - ref) / np.linalg.norm(ref)
            assert err < (2e-3 if dtype == torch.float32 else 2e-2)


SUBM_CASES = [
    # name, batches, shape, n, coordinate dtype, kernel, dilation
    ("small-box", 3, (37, 21, 13), 4000, torch.int16, 3, 1),
    ("dense", 2, (12, 12, 12), 3000, torch.int32, 3, 1),
    ("k5", 2, (30, 30, 30), 5000, torch.int16, 5, 1),
    ("dilated", 2, (30, 30, 30), 5000, torch.int16, 3, 2),
    ("one-voxel-box", 1, (1, 1, 1), 1, torch.int16, 3, 1),
    ("wide", 4, (1440, 1440, 41), 60000, torch.int16, 3, 1),
    ("int64", 2, (40, 50, 60), 6000, torch.int64, 3, 1),
    # 33.5M bricks: 2048 prefix tiles, above the count whose tile sums are scanned by a launch of
    # their own instead of summed inline by every workgroup
    ("many-tiles", 8, (2048, 2048, 64), 500000, torch.int16, 3, 1),
]


@pytest.mark.parametrize("case", SUBM_CASES, ids=[c[0] for c in SUBM_CASES])
def test_subm_brick_index_map_exact(device, case):
    """st_kmap_subm (brick index + query, one cooperative launch) equals the exact map, the hash-table
    query and the row masks, on boxes with partial bricks, dense sets, k = 5 and dilation 2."""
    from sparsetriton_amd.nn.functional.conv.kmap import subm_kernel_map
    name, B, shape, n, dt, k, d = case
    rng = np.random.default_rng(len(name) * 31 + n)
    vol = B * shape[0] * shape[1] * shape[2]
    lin = np.sort(rng.choice(vol, min(n, vol), replace=False))
    sx, sy, sz = shape
    c = np.stack([lin // (sx * sy * sz), (lin // (sy * sz)) % sx, (lin // sz) % sy, lin % sz], 1).astype(np.int32)
    coords = torch.as_tensor(c, dtype=dt, device=device)
    offs = _target_offsets(k, d, (k - 1) * d // 2, False, device)
    km, snap = subm_kernel_map(coords, B, shape, offs)
    expect = O.exact_kmap(c, c, O.target_offsets(k, d, (k - 1) * d // 2, False), 1, shape)
    assert (km.neighbor_indices.cpu().numpy() == expect).all()
    _check_masks(km)
    assert snap.counters() == {"overflow": 0, "bad_coord": 0, "duplicate": 0, "out_of_box": 0}
    assert km.symmetric == (k % 2 == 1)
    # the hash-table path gives the same map
    sp = SparseTensor(torch.zeros((c.shape[0], 1), device=device), coords, spatial_shape=shape, batch_size=B)
    table = _input_table(sp, 1)
    hashed = query_kernel_map(table, sp.C, offs, shape, 1, c.shape[0])
    assert torch.equal(hashed.nbr, km.nbr) and torch.equal(hashed.out_masks, km.out_masks)


def test_subm_brick_index_out_of_box_and_repeats(device):
    """Rows outside the box keep their in-box neighbours; repeats resolve to the lowest row; the
    status counts both (and the map is then not treated as its own transpose)."""
    from sparsetriton_amd.nn.functional.conv.kmap import subm_kernel_map
    rng = np.random.default_rng(88)
    c = _rand_coords(rng, 3000, 20)
    shape = (15, 18, 20)
    c[rng.choice(3000, 40, replace=False)] = c[rng.choice(3000, 40, replace=False)]
    coords = torch.as_tensor(c, dtype=torch.int16, device=device)
    offs = _target_offsets(3, 1, 1, False, device)
    km, snap = subm_kernel_map(coords, 2, shape, offs)
    expect = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, shape)
    assert (km.neighbor_indices.cpu().numpy() == expect).all()
    oob = ~((c[:, 1] < 15) & (c[:, 2] < 18))
    cnt = snap.counters()
    assert cnt["out_of_box"] == int(oob.sum()) and cnt["duplicate"] > 0 and cnt["bad_coord"] == 0
    assert not km.symmetric


def test_subm_brick_index_bad_coordinates(device):
    """int32 coordinates beyond the 16-bit key range (inside a box up to 65536 wide) are counted as
    unkeyable, and sparse_conv3d raises for them."""
    from sparsetriton_amd.nn.functional.conv.kmap import subm_kernel_map
    c = np.array([[0, 40000, 1, 1], [0, 40001, 1, 1], [0, 5, 5, 5]], dtype=np.int32)
    coords = torch.as_tensor(c, device=device)
    km, snap = subm_kernel_map(coords, 1, (40002, 8, 8), _target_offsets(3, 1, 1, False, device))
    assert snap.counters()["bad_coord"] == 2


def test_subm_brick_index_declines_a_box_far_larger_than_the_set(device):
    """More than 64 bricks a row (plus slack): no brick index -- sparse_conv3d takes the hash table
    and gives the same exact map."""
    from sparsetriton_amd.nn.functional.conv.kmap import subm_kernel_map
    rng = np.random.default_rng(3)
    c = np.stack([np.zeros(500, np.int64), rng.integers(0, 4000, 500), rng.integers(0, 4000, 500),
                  rng.integers(0, 400, 500)], 1).astype(np.int32)
    c = np.unique(c, axis=0)
    coords = torch.as_tensor(c, dtype=torch.int16, device=device)
    offs = _target_offsets(3, 1, 1, False, device)
    assert subm_kernel_map(coords, 1, (4000, 4000, 400), offs) is None
    sp = SparseTensor(torch.randn((c.shape[0], 4), device=device), coords, spatial_shape=(4000, 4000, 400),
                      batch_size=1)
    out = sparse_conv3d(sp, torch.randn((27, 4, 4), device=device), 3)
    km = sp._cache.neighbor_indices[(3, 1, 1, 1, True, False)][1]
    assert (km.neighbor_indices.cpu().numpy() == O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1,
                                                             (4000, 4000, 400))).all()
    assert out.F.shape == (c.shape[0], 4)


def test_subm_brick_index_empty(device):
    from sparsetriton_amd.nn.functional.conv.kmap import subm_kernel_map
    coords = torch.empty((0, 4), dtype=torch.int16, device=device)
    km, snap = subm_kernel_map(coords, 1, (8, 8, 8), _target_offsets(3, 1, 1, False, device))
    assert km.nbr.shape == (27, 0)


def test_config5_subm_brick_index_exact(device):
    from sparsetriton_amd.nn.functional.conv.kmap import subm_kernel_map
    c, shape = workloads.config5()
    coords = torch.as_tensor(c, dtype=torch.int16, device=device)
    km, snap = subm_kernel_map(coords, 1, shape, _target_offsets(3, 1, 1, False, device))
    expect = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, shape)
    assert (km.neighbor_indices.cpu().numpy() == expect).all()
    assert km.symmetric


def test_gather_without_sources_writes_zeros(device):
    """A gather-GEMM over zero source rows (e.g. the input gradient of a layer whose output is
    empty) writes zero rows without touching the (storage-less) source array."""
    from sparsetriton_amd.nn.functional.conv.funcs.implicit_precomputed_gemm import gather_gemm, gather_gemm_tiled
    from sparsetriton_amd.nn.functional.conv.kmap import TileMap, TilePlan
    K, n_dst = 27, 300
    nbr = torch.full((K, n_dst), -1, dtype=torch.int32, device=device)
    masks = torch.zeros((n_dst, 1), dtype=torch.int32, device=device)
    perm = TilePlan.build(n_dst, K, masks).perm
    tiles = TileMap.build(nbr, n_dst, 1, masks, K, perm, n_dst, 0)
    assert int(tiles.nk.sum()) == 0
    for dt in (torch.float32, torch.bfloat16):
        A = torch.empty((0, 64), dtype=dt, device=device)
        Bt = torch.randn((K, 64, 64), device=device).to(dt)
        for out in (gather_gemm_tiled(A, tiles, Bt, n_dst, K), gather_gemm(A, nbr, n_dst, 1, masks, Bt, n_dst, K)):
            assert out.shape == (n_dst, 64) and int(torch.count_nonzero(out)) == 0


@pytest.mark.parametrize("spin", ["0", "1"])
def test_index_level_without_published_totals(device, spin, monkeypatch):
    """The one-launch index levels (counts + prefix) take the earlier tiles' totals as they are
    published, and compute any still missing after ST_SUBM_SPIN polls from the index itself.  With
    0 or 1 polls (nearly every total computed directly) the submanifold map, its masks and the
    strided brick build equal those of the default run."""
    from sparsetriton_amd.nn.functional.conv.kmap import subm_kernel_map
    rng = np.random.default_rng(41)
    B, shape, n = 4, (1440, 1440, 41), 60000
    vol = B * shape[0] * shape[1] * shape[2]
    lin = np.sort(rng.choice(vol, n, replace=False))
    sx, sy, sz = shape
    c = np.stack([lin // (sx * sy * sz), (lin // (sy * sz)) % sx, (lin // sz) % sy, lin % sz], 1).astype(np.int32)
    coords = torch.as_tensor(c, dtype=torch.int16, device=device)
    offs = _target_offsets(3, 1, 1, False, device)
    km0, _ = subm_kernel_map(coords, B, shape, offs)
    ref_strided = brick_out_coords_and_map(coords, B, shape, 3, 2, 1, 1, False)
    monkeypatch.setenv("ST_SUBM_SPIN", spin)
    km1, snap = subm_kernel_map(coords, B, shape, offs)
    got_strided = brick_out_coords_and_map(coords, B, shape, 3, 2, 1, 1, False)
    assert torch.equal(km0.nbr, km1.nbr) and torch.equal(km0.out_masks, km1.out_masks)
    assert snap.counters() == {"overflow": 0, "bad_coord": 0, "duplicate": 0, "out_of_box": 0}
    assert torch.equal(ref_strided[0], got_strided[0])
    assert torch.equal(ref_strided[3].nbr, got_strided[3].nbr)
    assert torch.equal(ref_strided[3].invnbr, got_strided[3].invnbr)
