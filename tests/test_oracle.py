"""Pins the CPU oracle (test infrastructure) before any GPU result is compared to it.

What pins each oracle function:
  exact_kmap      brute-force dictionary lookup (bf_kmap) on random sets, all geometries
  out_coords      brute-force candidate loop (same order) and, as a set, the nonzero
                  pattern of a dense convolution of the occupancy grid (golden fixtures)
  fwd/dgrad/wgrad dense conv3d / conv_transpose3d values and autograd gradients
                  (golden fixtures, torch float64)
  RefHash         the reference tests' known answers (tests/test_utils_hash.py:95-123)
                  and the closed-form key2 alias of (0,0,0,0) / (1,10,0,29)
  pool            torch max_pool3d / avg_pool3d of dense grids (empty cells -inf / uncounted)
                  where the cell rule is standard pooling (odd kernel, padding k // 2); the
                  cell rule for any kernel / padding by a search over cells
  pool_grad       torch autograd through the same dense max_pool3d / avg_pool3d
  ledger port     ref_out_coords equals the exact build where nothing aliases; every map
                  difference is traced to a key2 alias or a lost row (tests/test_ledger.py)
  *_f64_blas      equality with the loop versions (fwd/dgrad/wgrad_f64)
  upsample        the reference's own known answer (tests/test_pooling.py:14-40)
  batch_norm      torch.nn.functional.batch_norm applied sample by sample (outputs), the
                  unbiased/biased relation to torch's running variance (running statistics),
                  and central finite differences of the numpy forward (gradients)
A mistake such as a sign flip in t_k, a transposed weight operand or a wrong
stride rule breaks one of these.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLD = Path(__file__).resolve().parent / "golden"


def _rand_coords(rng, n, S=8, B=2):
    lin = np.sort(rng.choice(B * S ** 3, n, replace=False))
    return np.stack([lin // S ** 3, (lin // S ** 2) % S, (lin // S) % S, lin % S], 1).astype(np.int32)


GEOMS = [(3, 1, 1, 1, False), (3, 2, 1, 1, False), (5, 2, 2, 1, False), (3, 2, 1, 2, False), (3, 1, 0, 1, False),
         (3, 2, 1, 1, True), (3, 1, 1, 1, True), (3, 3, 0, 1, True), (2, 2, 0, 1, False)]


@pytest.mark.parametrize("k,s,p,d,tr", GEOMS)
def test_out_coords_and_kmap_vs_bruteforce(k, s, p, d, tr):
    rng = np.random.default_rng(k * 100 + s * 10 + p + d + tr)
    S = 8
    c = _rand_coords(rng, 70, S)
    off = O.target_offsets(k, d, p, tr)
    ns = O.out_shape((S, S, S), k, s, d, p, tr)
    oc = O.out_coords(c, off, s, tr, ns)
    ob = O.bf_out_coords(c, off, s, tr, ns)
    assert oc.shape == ob.shape and (oc == ob).all()
    if tr:
        a = O.exact_kmap(c, oc, off, 1, tuple(v * s for v in (S, S, S)), in_scale=s)
        b = O.bf_kmap(c, oc, off, 1, tuple(v * s for v in (S, S, S)), in_scale=s)
    else:
        a = O.exact_kmap(c, oc, off, s, (S, S, S))
        b = O.bf_kmap(c, oc, off, s, (S, S, S))
    assert (a == b).all()
    assert (a >= 0).sum() > 0


def test_subm_kmap_vs_bruteforce_with_out_of_bounds():
    rng = np.random.default_rng(7)
    c = _rand_coords(rng, 90, 8)
    off = O.target_offsets(3, 1, 1, False)
    # a spatial shape smaller than the coordinates: the bounds check must drop neighbours
    shape = (6, 7, 8)
    assert (O.exact_kmap(c, c, off, 1, shape) == O.bf_kmap(c, c, off, 1, shape)).all()


@pytest.mark.parametrize("case", ["in_box", "out_of_box", "duplicates"])
def test_subm_symmetric_gather_is_the_adjoint_only_when_clean(case):
    """The submanifold input-gradient shortcut -- gather dY through nbr[K-1-k, i] -- equals the
    scatter adjoint over the forward map (dgrad_f64, the reference's implicit_precomputed_gemm.py
    :129-177) exactly when every row is unique and inside the shape; otherwise it drops terms.
    The GEMM path may take it only under that condition."""
    rng = np.random.default_rng(9)
    n, S = 1500, 12
    c = _rand_coords(rng, n, S)
    shape = (9, 11, 12) if case == "out_of_box" else (S, S, S)
    if case == "duplicates":
        c[rng.choice(n, 40, replace=False)] = c[rng.choice(n, 40, replace=False)]
    off = O.target_offsets(3, 1, 1, False)
    nbr = O.exact_kmap(c, c, off, 1, shape)
    X = rng.standard_normal((n, 5))
    W = rng.standard_normal((27, 5, 6))
    dY = rng.standard_normal((n, 6))
    scatter = O.dgrad_f64(dY, W, nbr, n)
    gather = np.zeros((n, 5))
    for k in range(27):
        o = nbr[:, 26 - k]
        ok = o >= 0
        gather[ok] += dY[o[ok]] @ W[k].T
    err = np.abs(gather - scatter).max()
    if case == "in_box":
        assert err < 1e-9
    else:
        assert err > 1e-3
    # adjoint identity of the oracle pair itself: <dY, fwd(X)> = <dgrad(dY), X>
    assert abs((dY * O.fwd_f64(X, W, nbr)).sum() - (scatter * X).sum()) < 1e-8 * n


@pytest.mark.parametrize("dup", [False, True])
def test_blas_gemms_equal_the_loop_oracle(dup):
    """The per-offset BLAS restatements (benchmark-size checkers) equal the pinned loop
    versions, including maps with absent entries and an input row repeated within an offset."""
    rng = np.random.default_rng(12)
    n_in, n_out, K = 300, 260, 27
    nbr = rng.integers(-1, n_in, (n_out, K)).astype(np.int32)
    nbr[rng.random((n_out, K)) < 0.6] = -1
    if dup:
        nbr[5, 3] = nbr[9, 3] = 17
    X = rng.standard_normal((n_in, 6))
    W = rng.standard_normal((K, 6, 7))
    dY = rng.standard_normal((n_out, 7))
    assert np.allclose(O.fwd_f64_blas(X, W, nbr), O.fwd_f64(X, W, nbr), rtol=1e-12, atol=1e-12)
    assert np.allclose(O.dgrad_f64_blas(dY, W, nbr, n_in), O.dgrad_f64(dY, W, nbr, n_in), rtol=1e-12, atol=1e-12)
    assert np.allclose(O.wgrad_f64_blas(X, dY, nbr, K), O.wgrad_f64(X, dY, nbr, K), rtol=1e-12, atol=1e-12)


def _cases():
    z = np.load(GOLD / "conv_cases.npz")
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


@pytest.mark.parametrize("name", _cases()[1])
def test_oracle_vs_dense_golden(name):
    z, _ = _cases()
    g = lambda key: z[f"{name}/{key}"]
    C_in, C_out, k, s, p, d, tr, subm = (int(v) for v in g("meta"))
    c, X, W = g("coords"), g("feats").astype(np.float64), g("weight").astype(np.float64)
    S = tuple(int(v) for v in g("spatial_shape"))
    off = O.target_offsets(k, d, p, bool(tr))
    if subm:
        oc = c
    else:
        ns = O.out_shape(S, k, s, d, p, bool(tr))
        assert tuple(int(v) for v in g("out_shape")) == ns
        oc = O.out_coords(c, off, s, bool(tr), ns)
        # same set as the dense occupancy convolution
        key = lambda a: set(map(tuple, np.asarray(a).tolist()))
        assert key(oc) == key(g("out_coords"))
    if tr:
        nbr = O.exact_kmap(c, oc, off, 1, tuple(v * s for v in S), in_scale=s)
    else:
        nbr = O.exact_kmap(c, oc, off, s, S)
    # reorder golden rows to the oracle's output order
    gold_rows = {tuple(r): i for i, r in enumerate(g("out_coords").tolist())}
    perm = np.array([gold_rows[tuple(r)] for r in oc.tolist()])
    out = O.fwd_f64(X, W, nbr)
    np.testing.assert_allclose(out, g("out")[perm], rtol=1e-5, atol=1e-5)
    dY = g("dY").astype(np.float64)[perm]
    np.testing.assert_allclose(O.dgrad_f64(dY, W, nbr, c.shape[0]), g("dX"), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(O.wgrad_f64(X, dY, nbr, k ** 3), g("dW"), rtol=1e-5, atol=1e-5)


def test_ref_hash_port_reference_kats():
    kats = json.loads((GOLD / "reference_kats.json").read_text())
    for case in kats["hash_table"]["cases"]:
        h = O.RefHash(case["insert"], factor=case["capacity"] / len(case["insert"]))
        assert h.query(case["query"]).tolist() == case["expect"]


def test_ref_hash_port_alias_defect():
    kats = json.loads((GOLD / "reference_kats.json").read_text())["reference_hash_alias"]
    # capacity 5 puts both coordinates' probe chains on slot 0; key2 aliases, so the
    # reference's query returns row 0 for a coordinate that was never inserted.
    h = O.RefHash([kats["a"]], factor=5.0)
    assert h.T == 5
    assert h.query([kats["b"]]).tolist() == [0]


def test_ref_kmap_port_equals_exact_when_lossless():
    rng = np.random.default_rng(3)
    c = _rand_coords(rng, 200, 12)
    off = O.target_offsets(3, 1, 1, False)
    h = O.RefHash(c)
    assert h.dropped == 0
    ref = h.kmap(c, off, 1, (12, 12, 12))
    exact = O.exact_kmap(c, c, off, 1, (12, 12, 12))
    # the reference port may only differ by key2 aliasing; on this set it does not
    assert (ref == exact).mean() > 0.999


def test_ref_gemm_port_matches_f64():
    rng = np.random.default_rng(4)
    c = _rand_coords(rng, 150, 10)
    off = O.target_offsets(3, 1, 1, False)
    nbr = O.exact_kmap(c, c, off, 1, (10, 10, 10))
    X = rng.standard_normal((150, 6)).astype(np.float32)
    W = rng.standard_normal((27, 6, 10)).astype(np.float32)
    dY = rng.standard_normal((150, 10)).astype(np.float32)
    np.testing.assert_allclose(O.ref_fwd_f32(X, W, nbr), O.fwd_f64(X, W, nbr), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(O.ref_dgrad_f32(dY, W, nbr, 150), O.dgrad_f64(dY, W, nbr, 150), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(O.ref_wgrad_f32(X, dY, nbr, 27), O.wgrad_f64(X, dY, nbr, 27), rtol=1e-4, atol=1e-4)


def test_offset_convention_kat():
    kats = json.loads((GOLD / "reference_kats.json").read_text())["offset_convention"]
    t = O.target_offsets(3, 1, 1, False)
    assert list(t.shape) == kats["base_offsets_shape"]
    # submanifold: neighbour = out - t_k = out + base_k
    for key, k in kats["k_of"].items():
        base = [int(v) for v in key.split(",")]
        assert (-t[k]).tolist() == base


def test_product_offsets_match_oracle():
    from sparsetriton_amd.nn.functional.conv.kmap import _target_offsets
    for k, d, p, tr in [(3, 1, 1, False), (5, 2, 2, False), (3, 1, 1, True), (3, 1, 0, True), (2, 1, 0, False)]:
        assert (_target_offsets(k, d, p, tr, "cpu").numpy() == O.target_offsets(k, d, p, tr)).all()


def test_flatten_kats():
    from sparsetriton_amd.utils.hash import flatten_coord, unflatten_coord
    kats = json.loads((GOLD / "reference_kats.json").read_text())["flatten_coord"]
    for case in kats["cases"]:
        assert flatten_coord(torch.tensor(case["coords"])).tolist() == case["flat"]
    rt = torch.tensor(kats["roundtrip"])
    assert torch.equal(unflatten_coord(flatten_coord(rt)).long(), rt)


def test_hash_coords_helper():
    from sparsetriton_amd.utils.hash import hash_coords
    h = hash_coords(torch.tensor([[0, 1, 2, 3], [0, 1, 2, 4]]))
    assert h.dtype == torch.int32 and h.shape == (2,) and (h >= 0).all() and h[0] != h[1]
    assert torch.unique(hash_coords(torch.randint(0, 100, (1000, 4)))).shape[0] > 500
    # int32 wrap-around semantics, computed independently with numpy int32
    c = np.array([[3, 40000, 50000, 60000]], dtype=np.int32)
    with np.errstate(over="ignore"):
        ref = ((c[:, 1] * np.int32(73856093)) ^ (c[:, 2] * np.int32(19349663)) ^ (c[:, 3] * np.int32(83492791))
               ^ (c[:, 0] * np.int32(1000003))) & np.int32(0x7FFFFFFF)
    assert hash_coords(torch.as_tensor(c)).tolist() == ref.tolist()


# ------------------------------------------------------------ batch norm

def test_batch_norm_matches_library_per_sample():
    import torch.nn.functional as F

    rng = np.random.default_rng(7)
    x = rng.standard_normal((400, 6)) * 3 + 1
    bi = rng.integers(0, 4, 400)
    bi[bi == 2] = 3  # sample 2 has no rows
    w, b = rng.standard_normal(6), rng.standard_normal(6)
    res = rng.standard_normal((400, 6))
    out, rm, rv = O.batch_norm_f64(x, bi, 4, w, b, np.zeros(6), np.ones(6), True, residual=res, relu=True)
    for s in (0, 1, 3):
        r = bi == s
        ref = F.batch_norm(torch.tensor(x[r]), None, None, torch.tensor(w), torch.tensor(b), training=True).numpy()
        assert np.abs(out[r] - np.maximum(ref + res[r], 0)).max() < 1e-12
    # evaluation: the library routine with the running statistics
    rm0, rv0 = rng.standard_normal(6), rng.uniform(0.5, 2, 6)
    out_e, _, _ = O.batch_norm_f64(x, bi, 4, w, b, rm0, rv0, False)
    ref = F.batch_norm(torch.tensor(x), torch.tensor(rm0), torch.tensor(rv0), torch.tensor(w), torch.tensor(b),
                       training=False).numpy()
    assert np.abs(out_e - ref).max() < 1e-12


def test_batch_norm_running_stats_one_sample():
    import torch.nn.functional as F

    rng = np.random.default_rng(8)
    n, m = 50, 0.1
    x = rng.standard_normal((n, 5))
    rm0, rv0 = rng.standard_normal(5), rng.uniform(0.5, 2, 5)
    _, rm, rv = O.batch_norm_f64(x, np.zeros(n, np.int64), 1, None, None, rm0, rv0, True, momentum=m)
    trm, trv = torch.tensor(rm0), torch.tensor(rv0)
    F.batch_norm(torch.tensor(x), trm, trv, training=True, momentum=m)
    assert np.abs(rm - trm.numpy()).max() < 1e-12
    # torch moves towards the unbiased variance, the reference towards the biased one
    assert np.abs((rv - (1 - m) * rv0) - (trv.numpy() - (1 - m) * rv0) * (n - 1) / n).max() < 1e-12


@pytest.mark.parametrize("training,relu", [(True, True), (True, False), (False, True)])
def test_batch_norm_grads_finite_differences(training, relu):
    rng = np.random.default_rng(9)
    n, C, B = 24, 3, 2
    x = rng.standard_normal((n, C))
    bi = rng.integers(0, B, n)
    w, b = rng.standard_normal(C), rng.standard_normal(C)
    rm0, rv0 = rng.standard_normal(C), rng.uniform(0.5, 2, C)
    res = rng.standard_normal((n, C))
    dout = rng.standard_normal((n, C))
    dx, dw, db, dres = O.batch_norm_grads_f64(x, bi, B, w, b, rm0, rv0, training, dout, residual=res, relu=relu)

    def f(x_, w_, b_, r_):
        return float((O.batch_norm_f64(x_, bi, B, w_, b_, rm0, rv0, training, residual=r_, relu=relu)[0]
                      * dout).sum())

    h = 1e-6
    for (arr, g) in ((x, dx), (w, dw), (b, db), (res, dres)):
        num = np.zeros_like(arr)
        for i in np.ndindex(arr.shape):
            a0 = arr[i]
            arr[i] = a0 + h
            fp = f(x, w, b, res)
            arr[i] = a0 - h
            fm = f(x, w, b, res)
            arr[i] = a0
            num[i] = (fp - fm) / (2 * h)
        assert np.abs(num - g).max() < 1e-5 * max(1.0, np.abs(g).max())


# ------------------------------------------------------------ pooling, upsampling

@pytest.mark.parametrize("s", [2, 3])
@pytest.mark.parametrize("mode", ["max", "avg"])
def test_pool_matches_dense_library_pooling(s, mode):
    import torch.nn.functional as F

    rng = np.random.default_rng(s * 10 + len(mode))
    S = 12
    c = _rand_coords(rng, 300, S)
    f = rng.standard_normal((c.shape[0], 3))
    k, p = 3, 1  # odd kernel, padding k // 2: the cell of x is floor(x / s), standard pooling
    oc, out, inv = O.pool_f64(c, f, k, p, s, mode)
    B = int(c[:, 0].max()) + 1
    fill = -np.inf if mode == "max" else 0.0
    dense = torch.full((B, 3, S, S, S), fill, dtype=torch.float64)
    occ = torch.zeros((B, 1, S, S, S), dtype=torch.float64)
    ct = torch.as_tensor(c, dtype=torch.long)
    dense[ct[:, 0], :, ct[:, 1], ct[:, 2], ct[:, 3]] = torch.as_tensor(f)
    occ[ct[:, 0], 0, ct[:, 1], ct[:, 2], ct[:, 3]] = 1.0
    if mode == "max":
        ref = F.max_pool3d(dense, s, s, ceil_mode=True)
    else:
        ref = F.avg_pool3d(dense, s, s, ceil_mode=True) / F.avg_pool3d(occ, s, s, ceil_mode=True)
    o = torch.as_tensor(oc, dtype=torch.long)
    assert np.abs(out - ref[o[:, 0], :, o[:, 1], o[:, 2], o[:, 3]].numpy()).max() < 1e-12
    # every occupied cell is an output, in ascending order
    cnt = F.avg_pool3d(occ, s, s, ceil_mode=True) * s ** 3
    assert int((cnt > 0).sum()) == oc.shape[0]
    assert (np.lexsort(oc.T[::-1]) == np.arange(oc.shape[0])).all()
    assert (oc[inv] == np.concatenate([c[:, :1], c[:, 1:] // s], 1)).all()


@pytest.mark.parametrize("s", [2, 3])
@pytest.mark.parametrize("mode", ["max", "avg"])
def test_pool_grad_matches_dense_library_autograd(s, mode):
    """pool_grad_f64 (the reference's backward rule, spatial.py:139-209) equals torch autograd
    through dense max_pool3d / avg_pool3d of the occupancy grid (random floats: no ties)."""
    import torch.nn.functional as F

    rng = np.random.default_rng(s * 7 + len(mode))
    S, C = 12, 3
    c = _rand_coords(rng, 300, S)
    f = rng.standard_normal((c.shape[0], C))
    oc, out, inv = O.pool_f64(c, f, 3, 1, s, mode)
    dout = rng.standard_normal(out.shape)
    B = int(c[:, 0].max()) + 1
    ct = torch.as_tensor(c, dtype=torch.long)
    vals = torch.as_tensor(f).requires_grad_(True)
    base = torch.full((B, C, S, S, S), -np.inf if mode == "max" else 0.0, dtype=torch.float64)
    dense = base.clone()
    dense[ct[:, 0], :, ct[:, 1], ct[:, 2], ct[:, 3]] = vals
    occ = torch.zeros((B, 1, S, S, S), dtype=torch.float64)
    occ[ct[:, 0], 0, ct[:, 1], ct[:, 2], ct[:, 3]] = 1.0
    if mode == "max":
        pooled = F.max_pool3d(dense, s, s, ceil_mode=True)
    else:
        pooled = F.avg_pool3d(dense, s, s, ceil_mode=True) / F.avg_pool3d(occ, s, s, ceil_mode=True).clamp_min(1e-30)
    o = torch.as_tensor(oc, dtype=torch.long)
    sel = pooled[o[:, 0], :, o[:, 1], o[:, 2], o[:, 3]]
    (sel * torch.as_tensor(dout)).sum().backward()
    assert np.abs(O.pool_grad_f64(f, out, inv, dout, mode) - vals.grad.numpy()).max() < 1e-12


@pytest.mark.parametrize("k,p,s", [(2, 0, 2), (2, 1, 2), (4, 1, 2), (4, 2, 3), (3, 0, 2), (3, 2, 2), (1, 0, 1)])
def test_pool_cell_rule_by_search(k, p, s):
    """Cells for even kernels and any padding (negative cells included) equal a search for the
    one cell o with o * s <= x + p - k // 2 < (o + 1) * s (spatial.py:118-119), so a truncating
    division or a dropped term cannot pass."""
    rng = np.random.default_rng(k * 100 + p * 10 + s)
    c = _rand_coords(rng, 200, 9)
    oc, _, inv = O.pool_f64(c, rng.standard_normal((c.shape[0], 1)), k, p, s, "avg")
    for r in range(c.shape[0]):
        want = [c[r, 0]]
        for a in range(1, 4):
            v = int(c[r, a]) + p - k // 2
            o = next(o for o in range(-10, 20) if o * s <= v < (o + 1) * s)
            want.append(o)
        assert list(oc[inv[r]]) == want
    if k // 2 > p:
        assert (oc[:, 1:] < 0).any()  # the rule sends coordinate 0 to a negative cell here


def test_torch_f64_compositions_equal_the_numpy_oracle():
    """conv_f64_torch / batch_norm_f64_torch (the differentiable block / backbone checkers) equal
    fwd_f64 and batch_norm_f64, and their autograd equals dgrad_f64 / wgrad_f64 /
    batch_norm_grads_f64."""
    rng = np.random.default_rng(17)
    c = _rand_coords(rng, 200, 8)
    nbr = O.exact_kmap(c, c, O.target_offsets(3, 1, 1, False), 1, (8, 8, 8))
    X, W, dY = rng.standard_normal((200, 4)), rng.standard_normal((27, 4, 5)), rng.standard_normal((200, 5))
    x = torch.tensor(X, requires_grad=True)
    w = torch.tensor(W, requires_grad=True)
    y = O.conv_f64_torch(x, w, None, nbr)
    y.backward(torch.as_tensor(dY))
    assert np.abs(y.detach().numpy() - O.fwd_f64(X, W, nbr)).max() < 1e-12
    assert np.abs(x.grad.numpy() - O.dgrad_f64(dY, W, nbr, 200)).max() < 1e-12
    assert np.abs(w.grad.numpy() - O.wgrad_f64(X, dY, nbr, 27)).max() < 1e-12
    bi = c[:, 0]
    g, bb, res = rng.uniform(0.5, 1.5, 5), rng.standard_normal(5), rng.standard_normal((200, 5))
    yt = torch.tensor(O.fwd_f64(X, W, nbr), requires_grad=True)
    z = O.batch_norm_f64_torch(yt, bi, 2, torch.as_tensor(g), torch.as_tensor(bb), torch.as_tensor(res), relu=True)
    ref, _, _ = O.batch_norm_f64(yt.detach().numpy(), bi, 2, g, bb, np.zeros(5), np.ones(5), True, residual=res,
                                 relu=True)
    assert np.abs(z.detach().numpy() - ref).max() < 1e-12
    z.backward(torch.as_tensor(dY))
    gx = O.batch_norm_grads_f64(yt.detach().numpy(), bi, 2, g, bb, np.zeros(5), np.ones(5), True, dY, residual=res,
                                relu=True)[0]
    assert np.abs(yt.grad.numpy() - gx).max() < 1e-12


def test_upsample_reference_kat():
    # tests/test_pooling.py:14-40: one voxel at the origin, s in 1..3
    for s in (1, 2, 3):
        oc, of = O.upsample_f64(np.array([[0, 0, 0, 0]]), np.array([[1.0, 2.0, 3.0]]), s)
        assert oc.shape == (s ** 3, 4) and (of == [1.0, 2.0, 3.0]).all()
        expect = [[0, x, y, z] for x in range(s) for y in range(s) for z in range(s)]
        assert oc.tolist() == expect
