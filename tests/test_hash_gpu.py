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


def _occupancy_np(c, B, shape):
    """Bitmap in the documented brick layout: bit (x%4)*16+(y%4)*4+z%4 of word ((b*BX+x/4)*BY+y/4)*BZ+z/4."""
    BX, BY, BZ = ((s + 3) // 4 for s in shape)
    words = np.zeros(B * BX * BY * BZ, dtype=np.uint64)
    inside = ((c[:, 0] >= 0) & (c[:, 0] < B) & (c[:, 1] >= 0) & (c[:, 1] < shape[0]) & (c[:, 2] >= 0)
              & (c[:, 2] < shape[1]) & (c[:, 3] >= 0) & (c[:, 3] < shape[2]))
    b, x, y, z = (c[inside, j].astype(np.int64) for j in range(4))
    w = ((b * BX + x // 4) * BY + y // 4) * BZ + z // 4
    bit = ((x % 4) * 16 + (y % 4) * 4 + z % 4).astype(np.uint64)
    np.bitwise_or.at(words, w, np.uint64(1) << bit)
    return words


@pytest.mark.parametrize("shape", [(37, 21, 13), (64, 64, 64), (1, 1, 1)])
def test_occupancy_bitmap_layout(device, shape):
    rng = np.random.default_rng(sum(shape))
    B = 3
    n = min(5000, B * shape[0] * shape[1] * shape[2] // 2 + 1)
    c = np.stack([rng.integers(0, B, n), rng.integers(0, shape[0], n), rng.integers(0, shape[1], n),
                  rng.integers(0, shape[2], n)], 1)
    c = np.concatenate([c, [[0, shape[0], 0, 0], [B, 0, 0, 0]]])  # outside the box: not in the bitmap
    t = HashTable(capacity=2 * c.shape[0], device=device)
    ct = torch.tensor(c, dtype=torch.int32, device=device)
    t.insert(ct)
    assert t.build_occupancy(ct, B, shape)
    got = t.occupancy[0].cpu().numpy().view(np.uint64)
    assert np.array_equal(got, _occupancy_np(c, B, shape))
    # rank index: prefix = exclusive popcount prefix of the words; rowmap[rank] = lowest row
    # of the rank-th set voxel in word / bit order
    prefix, rowmap = (x.cpu().numpy() for x in t.occupancy[2][1:3])
    pcs = np.array([bin(int(v)).count("1") for v in got], dtype=np.int64)
    assert np.array_equal(prefix, np.concatenate([[0], np.cumsum(pcs)]))
    BX, BY, BZ = ((s + 3) // 4 for s in shape)
    inside = (c[:, 0] < B) & (c[:, 1] < shape[0])
    ci = c[inside].astype(np.int64)
    rows = np.nonzero(inside)[0]
    lin = (((ci[:, 0] * BX + ci[:, 1] // 4) * BY + ci[:, 2] // 4) * BZ + ci[:, 3] // 4) * 64 + \
        (ci[:, 1] % 4) * 16 + (ci[:, 2] % 4) * 4 + ci[:, 3] % 4
    uniq, first = np.unique(lin, return_index=True)  # sorted = rank order; first = lowest row (rows ascend)
    assert np.array_equal(rowmap[:len(uniq)], rows[first])
    # rebuilding over other coordinates clears the previous bits
    half = c.shape[0] // 2
    assert t.build_occupancy(ct[:half], B, shape)
    assert np.array_equal(t.occupancy[0].cpu().numpy().view(np.uint64), _occupancy_np(c[:half], B, shape))
    t.clear()
    assert t.occupancy is None


def test_occupancy_size_rule(device):
    t = HashTable(capacity=64, device=device)
    c = torch.tensor([[0, 1, 2, 3]], dtype=torch.int32, device=device)
    t.insert(c)
    # a 4096^3 box for one voxel is far more than the probes it would save: not built
    assert not t.build_occupancy(c, 1, (4096, 4096, 4096))
    assert t.occupancy is None and t.occupancy_ref() is None
    assert t.build_occupancy(c, 1, (8, 8, 8))
