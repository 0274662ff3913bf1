"""GPU coordinate hash table vs exact lookups (bit-exact), including the reference's KATs."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from sparsetriton_amd.utils.hash import HashTable

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def test_reference_kats(device):
    kats = json.loads((GOLD / "reference_kats.json").read_text())["hash_table"]["cases"]
    for case in kats:
        t = HashTable(capacity=case["capacity"], device=device)
        assert t.capacity == case["capacity"]
        assert torch.all(t.table_keys == -1) and torch.all(t.table_values == -1)
        t.insert(torch.tensor(case["insert"], dtype=torch.int32, device=device))
        assert torch.any(t.table_keys != -1)
        assert t.query(torch.tensor(case["query"], dtype=torch.int32, device=device)).tolist() == case["expect"]
        t.check()


@pytest.mark.parametrize("dtype", [torch.int16, torch.int32, torch.int64])
def test_random_insert_query_exact(device, dtype):
    rng = np.random.default_rng(11)
    n = 200_000
    lin = rng.choice(4 * 512 * 512 * 64, n, replace=False)
    c = np.stack([lin // (512 * 512 * 64), (lin // (512 * 64)) % 512, (lin // 64) % 512, lin % 64], 1)
    miss = np.stack([rng.integers(0, 4, n), rng.integers(0, 512, n), rng.integers(0, 512, n),
                     rng.integers(64, 128, n)], 1)  # z >= 64: never inserted
    q = np.concatenate([c, miss])
    perm = rng.permutation(q.shape[0])
    q = q[perm]
    expect = np.concatenate([np.arange(n), np.full(n, -1)])[perm]
    t = HashTable(capacity=2 * n, device=device)
    t.insert(torch.as_tensor(c, dtype=dtype, device=device))
    t.check()
    got = t.query(torch.as_tensor(q, dtype=dtype, device=device)).cpu().numpy()
    assert (got == expect).all()
    # exactly n occupied slots, each key the packed coordinate of its value's row
    keys = t.table_keys.cpu().numpy()
    vals = t.table_values.cpu().numpy()
    occ = keys != -1
    assert occ.sum() == n
    packed = (c[:, 0].astype(np.int64) << 48) | (c[:, 1].astype(np.int64) << 32) | (c[:, 2] << 16) | c[:, 3]
    assert (keys[occ] == packed[vals[occ]]).all()


def test_full_table_and_overflow(device):
    c = torch.tensor([[0, i, 0, 0] for i in range(15)], dtype=torch.int32, device=device)
    t = HashTable(capacity=10, device=device)
    t.insert(c[:10])  # exactly full: no overflow
    assert t.counters()["overflow"] == 0
    assert t.query(c[:10]).tolist() == list(range(10))
    assert t.query(c[10:]).tolist() == [-1] * 5  # full sweep of a full table terminates
    t.insert(c[10:])
    assert t.counters()["overflow"] == 5
    with pytest.raises(RuntimeError, match="full"):
        t.check()


def test_capacity_assert():
    t = HashTable(capacity=10, device="cpu")
    with pytest.raises(AssertionError, match="capacity should be at least"):
        t.insert(torch.randint(0, 10, (20, 4), dtype=torch.int32))


def test_duplicates_resolve_to_lowest_row(device):
    c = torch.tensor([[0, 1, 1, 1], [0, 2, 2, 2], [0, 1, 1, 1], [0, 1, 1, 1], [0, 2, 2, 2]], dtype=torch.int32,
                     device=device)
    for _ in range(3):
        t = HashTable(capacity=64, device=device)
        t.insert(c)
        assert t.query(c).tolist() == [0, 1, 0, 0, 1]
        assert t.counters()["duplicate"] == 3


def test_many_duplicates_resolve_to_lowest_row(device):
    """Every key repeated three times across the whole launch (copies in shuffled order after the
    originals): whichever row's CAS claims a slot, the table ends with the key's lowest row."""
    rng = np.random.default_rng(7)
    n = 60_000
    lin = rng.choice(4 * 128 ** 3, n, replace=False)
    c = np.stack([lin // 128 ** 3, (lin // 128 ** 2) % 128, (lin // 128) % 128, lin % 128], 1)
    allc = np.concatenate([c, c[rng.permutation(n)], c[::-1]])
    t = HashTable(capacity=3 * n, device=device)
    t.insert(torch.as_tensor(allc, dtype=torch.int32, device=device))
    assert t.counters()["duplicate"] == 2 * n
    got = t.query(torch.as_tensor(c, dtype=torch.int32, device=device)).cpu().numpy()
    assert (got == np.arange(n)).all()


def test_unpackable_coordinates(device):
    c = torch.tensor([[0, 40000, 0, 0], [-1, 0, 0, 0], [0, 5, 5, 5]], dtype=torch.int32, device=device)
    t = HashTable(capacity=16, device=device)
    t.insert(c)
    assert t.counters()["bad_coord"] == 2
    with pytest.raises(RuntimeError, match="packable"):
        t.check()
    assert t.query(c).tolist() == [-1, -1, 2]


def test_reference_alias_pair_is_not_confused(device):
    # key2 of these two coordinates collides in the reference's table (hash.py:136-152);
    # exact keys keep them apart even when both probe chains start on the same slot.
    kats = json.loads((GOLD / "reference_kats.json").read_text())["reference_hash_alias"]
    t = HashTable(capacity=5, device=device)
    t.insert(torch.tensor([kats["a"]], dtype=torch.int32, device=device))
    assert t.query(torch.tensor([kats["a"], kats["b"]], dtype=torch.int32, device=device)).tolist() == [0, -1]


def test_scaled_insert(device):
    c = torch.tensor([[0, 1, 2, 3], [1, 4, 5, 6]], dtype=torch.int16, device=device)
    t = HashTable(capacity=16, device=device)
    t.insert(c, scale=2)
    q = torch.tensor([[0, 2, 4, 6], [1, 8, 10, 12], [0, 1, 2, 3]], dtype=torch.int16, device=device)
    assert t.query(q).tolist() == [0, 1, -1]


def test_empty(device):
    t = HashTable(capacity=4, device=device)
    t.insert(torch.empty((0, 4), dtype=torch.int16, device=device))
    assert t.query(torch.empty((0, 4), dtype=torch.int16, device=device)).shape == (0,)


@pytest.fixture
def group_probes():
    """Switch the table's probes to 16-lane groups for one test (st_hash_probe_mode)."""
    from sparsetriton_amd import _lib
    fn = _lib.lib().st_hash_probe_mode
    prev = fn(1)
    yield
    fn(prev)


def test_group_probes_exact(device, group_probes):
    """The 16-lane group probes (insert, query, kernel-map query) give the per-thread probes'
    answers: exact lookups, duplicates counted, a full table terminating, the map bit-exact."""
    from oracle import oracle as O
    from sparsetriton_amd.nn.functional.conv.kmap import _target_offsets, query_kernel_map
    rng = np.random.default_rng(12)
    n = 100_000
    lin = rng.choice(2 * 256 * 256 * 32, n, replace=False)
    c = np.stack([lin // (256 * 256 * 32), (lin // (256 * 32)) % 256, (lin // 32) % 256, lin % 32], 1)
    miss = np.stack([rng.integers(0, 2, n), rng.integers(0, 256, n), rng.integers(0, 256, n),
                     rng.integers(32, 64, n)], 1)
    t = HashTable(capacity=2 * n, device=device)
    t.insert(torch.as_tensor(np.concatenate([c, c[:500]]), dtype=torch.int32, device=device))
    assert t.counters()["duplicate"] == 500
    got = t.query(torch.as_tensor(np.concatenate([c, miss]), dtype=torch.int32, device=device)).cpu().numpy()
    assert (got == np.concatenate([np.arange(n), np.full(n, -1)])).all()
    full = HashTable(capacity=10, device=device)
    cf = torch.tensor([[0, i, 0, 0] for i in range(15)], dtype=torch.int32, device=device)
    full.insert(cf[:10])
    assert full.counters()["overflow"] == 0
    assert full.query(cf).tolist() == list(range(10)) + [-1] * 5
    # kernel map through the group probes == the exact map
    cs = c[:20_000].copy()
    cs[:, 1:] %= 24
    _, keep = np.unique(cs, axis=0, return_index=True)
    cs = cs[np.sort(keep)].astype(np.int32)
    tab = HashTable(capacity=2 * cs.shape[0], device=device)
    tab.insert(torch.as_tensor(cs, device=device))
    offs = _target_offsets(3, 1, 1, False, device)
    km = query_kernel_map(tab, torch.as_tensor(cs, device=device), offs, (24, 24, 24), 1, cs.shape[0])
    want = O.exact_kmap(cs, cs, O.target_offsets(3, 1, 1, False), 1, (24, 24, 24))
    assert np.array_equal(km.neighbor_indices.cpu().numpy(), want)


@pytest.mark.parametrize("load", [0.5, 0.97])
def test_partitioned_build_spills_and_second_insert(device, load):
    """The partitioned build (st_hash_build) at a high load factor, where many probes run past
    their segment and finish by global CAS, then a second insert into the filled table (rows that
    repeat earlier keys and new ones): every key maps to its lowest row, repeats are counted, the
    table holds each key once and stays a valid linear-probing table (every query answers)."""
    rng = np.random.default_rng(int(load * 100))
    n1, n2 = 40_000, 5_000
    cap = int((n1 + n2) / load)
    lin = rng.choice(2 * 256 ** 3, n1 + n2, replace=False)
    c = np.stack([lin // 256 ** 3, (lin // 256 ** 2) % 256, (lin // 256) % 256, lin % 256], 1).astype(np.int32)
    first = c[:n1]
    # the second insert: 2,000 keys of the first, then n2 new keys
    pick = rng.choice(n1, 2_000, replace=False)
    second = np.concatenate([first[pick], c[n1:]])
    t = HashTable(capacity=cap, device=device)
    t.insert(torch.as_tensor(first, device=device))
    t.insert(torch.as_tensor(second, device=device))
    t.check()
    assert t.counters()["duplicate"] == 2_000
    got = t.query(torch.as_tensor(c, device=device)).cpu().numpy()
    # a key's value: the lowest row it was inserted with (row indices of either insert, as the
    # CAS insert keeps them: a repeat takes the minimum)
    expect = np.concatenate([np.arange(n1), 2_000 + np.arange(n2)])
    expect[pick] = np.minimum(expect[pick], np.arange(2_000))
    assert (got == expect).all()
    keys = t.table_keys.cpu().numpy()
    assert (keys != -1).sum() == n1 + n2
    assert np.unique(keys[keys != -1]).shape[0] == n1 + n2


def test_partitioned_build_equals_cas_insert(device):
    """st_hash_build and st_hash_insert (the CAS build) give the same key -> row mapping, status
    counts included, on a set with repeated and unpackable coordinates."""
    from sparsetriton_amd import _lib
    rng = np.random.default_rng(21)
    n = 100_000
    lin = rng.choice(4 * 512 * 512 * 64, n, replace=False)
    c = np.stack([lin // (512 * 512 * 64), (lin // (512 * 64)) % 512, (lin // 64) % 512, lin % 64], 1)
    c = np.concatenate([c, c[rng.choice(n, 3_000, replace=False)], [[0, 40000, 1, 1], [-1, 0, 0, 0]]])
    coords = torch.as_tensor(c.astype(np.int32), device=device)
    built = HashTable(capacity=2 * c.shape[0], device=device)
    built.insert(coords)
    cas = HashTable(capacity=2 * c.shape[0], device=device)
    prev = _lib.lib().st_hash_probe_mode(-1)
    assert prev == 0
    cas._materialize()
    _lib.fill_(cas._keys, -1)
    _lib.fill_(cas._vals, -1)
    _lib.call("st_hash_insert", _lib.ptr(coords), _lib.coord_code(coords.dtype), coords.shape[0], 1,
              _lib.ptr(cas._keys), _lib.ptr(cas._vals), cas.capacity, _lib.ptr(cas._status()),
              _lib.stream_of(coords.device))
    assert built.counters() == cas.counters()
    assert torch.equal(built.query(coords), cas.query(coords))
    kb, vb = built.table_keys.cpu().numpy(), built.table_values.cpu().numpy()
    kc, vc = cas.table_keys.cpu().numpy(), cas.table_values.cpu().numpy()
    ob, oc = np.argsort(kb), np.argsort(kc)
    assert np.array_equal(kb[ob], kc[oc]) and np.array_equal(vb[ob], vc[oc])
