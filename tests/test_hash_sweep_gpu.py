"""Seeded random sweep of the coordinate table (reference ``utils/hash.py:193-366``) against a
Python dict: sizes from 1 to 60,000 rows, capacities from barely above the distinct-key count to
4x (never below the row count, which the reference asserts), repeated coordinates (a key keeps its lowest row), negative and large coordinates inside the
packable range, int16 / int32 / int64 coordinates, per-thread and 16-lane probes, fresh builds
and inserts into a table that already holds keys; every query answered exactly (-1 for absent
keys), and an insert past the capacity reported."""
import numpy as np
import pytest
import torch

from sparsetriton_amd import _lib
from sparsetriton_amd.utils.hash import HashTable

pytestmark = pytest.mark.gpu


def _keys(c: np.ndarray) -> list:
    return [tuple(int(v) for v in r) for r in c]


@pytest.mark.parametrize("seed", range(200))
def test_hash_table_sweep(device, seed):
    rng = np.random.default_rng(80_000 + seed)
    n = int(rng.choice([1, 7, 100, 1000, 5000, 60000]))
    lo, hi = (-300, 300) if rng.random() < 0.3 else (0, 1 << int(rng.integers(4, 15)))
    cdt = [torch.int16, torch.int32, torch.int64][int(rng.integers(0, 3))]
    c = np.stack([rng.integers(0, 4, n), rng.integers(lo, hi, n), rng.integers(lo, hi, n), rng.integers(lo, hi, n)],
                 1).astype(np.int64)
    if rng.random() < 0.4 and n >= 2:  # repeated coordinates
        m = max(1, n // 5)
        c[rng.choice(n, m, replace=False)] = c[rng.choice(n, m, replace=False)]
    first = {}
    for i, key in enumerate(_keys(c)):
        first.setdefault(key, i)
    distinct = len(first)
    # at least one slot per inserted row, as the reference asserts (hash.py:534)
    cap = max(n, int(distinct * float(rng.choice([1.02, 1.3, 2.0, 4.0]))) + 1)
    group = bool(rng.random() < 0.3)
    prev = _lib.lib().st_hash_probe_mode(1 if group else 0)
    try:
        t = HashTable(capacity=cap, device=device)
        split = rng.random() < 0.3 and n >= 4
        if split:  # two inserts: the second into a table that already holds the first's keys
            h = n // 2
            t.insert(torch.as_tensor(c[:h], device=device).to(cdt))
            t.table_keys  # applies the first insert
            t.insert(torch.as_tensor(c[h:], device=device).to(cdt))
        else:
            t.insert(torch.as_tensor(c, device=device).to(cdt))
        # queries: every inserted key, plus keys that are absent
        absent = np.stack([rng.integers(4, 8, 64), rng.integers(lo, hi, 64), rng.integers(lo, hi, 64),
                           rng.integers(lo, hi, 64)], 1).astype(np.int64)
        q = np.concatenate([c, absent])
        got = t.query(torch.as_tensor(q, device=device).to(cdt)).cpu().numpy()
    finally:
        _lib.lib().st_hash_probe_mode(prev)
    if split:
        # rows of the second insert are numbered from 0 in their own tensor
        h = n // 2
        exp_first = {}
        for i, key in enumerate(_keys(c[:h])):
            exp_first.setdefault(key, i)
        second = {}
        for i, key in enumerate(_keys(c[h:])):
            second.setdefault(key, i)
        expect = []
        for key in _keys(q):
            if key in exp_first and key in second:
                expect.append(min(exp_first[key], second[key]))
            elif key in exp_first:
                expect.append(exp_first[key])
            else:
                expect.append(second.get(key, -1))
    else:
        expect = [first.get(key, -1) for key in _keys(q)]
    assert np.array_equal(got, np.array(expect, dtype=got.dtype)), (seed, n, cap, str(cdt), group, split)
