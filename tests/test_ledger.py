"""Defect ledger of the reference's lossy coordinate hash on the seeded benchmark sets (CPU).

The reference stores a 31-bit hash (key2) of each coordinate instead of the coordinate
(utils/hash.py:136-152, used as the key at :240, :248), gives up after 128 probes (:211, :263)
and dedups strided / transposed outputs through the same key2 (nn/functional/conv/kmap.py:56-97).
This build keys on exact coordinates, so its maps equal the exact map; the reference's differ
wherever key2 aliases or a probe chain runs out.  The port of the reference algorithm
(oracle RefHash / ref_kmap / ref_out_coords) is pinned first -- it equals the exact functions
where nothing aliases, and every difference it reports is traced to its cause -- then its counts
on the seeded configurations are recorded (the same figures as the ledger table in the design
notes).  Inserts and candidates run one at a time in order; the GPU runs them in lockstep blocks,
so which of two colliding keys wins a slot can differ there.
"""

import numpy as np
import pytest

from oracle import oracle as O
from sparsetriton_amd import workloads


def _key2(c):
    c = np.asarray(c, dtype=np.int64)
    h = ((c[:, 0] * 1000003) & 0xFFFFFFFF) ^ ((c[:, 1] * 100003) & 0xFFFFFFFF) ^ ((c[:, 2] * 10007) & 0xFFFFFFFF) \
        ^ (c[:, 3] & 0xFFFFFFFF)
    return h & 0x7FFFFFFF


def _rand_coords(rng, n, S=12, B=2):
    lin = np.sort(rng.choice(B * S ** 3, n, replace=False))
    return np.stack([lin // S ** 3, (lin // S ** 2) % S, (lin // S) % S, lin % S], 1).astype(np.int32)


@pytest.mark.parametrize("k,s,p,tr", [(3, 2, 1, False), (3, 1, 1, False), (5, 2, 2, False), (3, 2, 1, True),
                                      (3, 1, 1, True), (2, 2, 0, False)])
def test_ref_out_coords_equals_exact_where_nothing_aliases(k, s, p, tr):
    """Candidate order, stride and range filters of the port equal the exact (pinned) build."""
    rng = np.random.default_rng(k + 10 * s + tr)
    c = _rand_coords(rng, 300)
    off = O.target_offsets(k, 1, p, tr)
    ns = O.out_shape((12, 12, 12), k, s, 1, p, tr)
    ref, exhausted = O.ref_out_coords(c, off, s, tr, ns)
    exact = O.out_coords(c, off, s, tr, ns)
    assert exhausted == 0 and ref.shape == exact.shape and (ref == exact).all()


def test_ref_dedup_loses_an_aliased_output():
    """(0,4,39,11) and (0,10,83,45) share key2 = 257542, and their probe starts h1 = 272139 and
    676653 agree modulo the dedup table of 2 * 3 * 27 = 162 slots: the second one's probe meets
    the first one's key and the reference drops it as a duplicate."""
    a, b = (0, 4, 39, 11), (0, 10, 83, 45)
    assert _key2(np.array([a, b])).tolist() == [257542, 257542]
    c = np.array([a, b, (0, 50, 50, 30)], dtype=np.int32)
    off = O.target_offsets(3, 1, 1, False)
    ns = (100, 100, 60)
    ref, _ = O.ref_out_coords(c, off, 1, False, ns)
    exact = O.out_coords(c, off, 1, False, ns)
    ref_rows = {tuple(r) for r in ref.tolist()}
    assert b in {tuple(r) for r in exact.tolist()} and b not in ref_rows and a in ref_rows
    led = O.ledger(c, ns, 3, 1, 1, False, submanifold=False)
    assert led["outputs_lost"] >= 1


def _explain(c, shape, led_nbr, exact, h, off):
    """Every mismatch of the port's map is a key2 alias (a false / wrong row whose coordinate has
    the query's key2) or a row the port's table lost (a missing row it cannot retrieve)."""
    o, k = np.nonzero(led_nbr != exact)
    q = c[o, 1:].astype(np.int64) - off[k]
    qc = np.concatenate([c[o, :1], q], axis=1)
    got, want = led_nbr[o, k], exact[o, k]
    present = got >= 0
    assert (_key2(c[got[present]]) == _key2(qc[present])).all()  # false / wrong: aliases
    missing = (want >= 0) & (got < 0)
    lost = h.query(c[want[missing]]) != want[missing]
    assert lost.all()  # missing: the row itself is not retrievable from the table
    return int((~present).sum()), int(present.sum())


def test_ref_kmap_mismatches_are_all_explained():
    for c, shape in (workloads.config1(seed=0), workloads.config5(seed=0)):
        off = O.target_offsets(3, 1, 1, False)
        h = O.RefHash(c)
        ref = h.kmap(c, off, 1, shape)
        exact = O.exact_kmap(c, c, off, 1, shape)
        _explain(c, shape, ref, exact, h, off)


LEDGER = {
    # config: (insert_dropped, outputs_lost, exact map entries, missing, false, wrong)
    "config1": (0, None, 4834, 0, 2, 0),
    "config2": (0, None, 2072662, 0, 0, 0),
    "config3": (0, 0, 1582203, 0, 0, 0),
    "config4": (0, 0, 14165235, 0, 0, 0),
    "config5": (608, None, 17980788, 10950, 0, 0),
}


@pytest.fixture(scope="module")
def sets():
    c2, s2 = workloads.config2(seed=0)
    ns3 = O.out_shape(s2, 3, 2, 1, 1, False)
    c3 = O.out_coords(c2, O.target_offsets(3, 1, 1, False), 2, False, ns3)
    return {"config1": (workloads.config1(seed=0), {}), "config2": ((c2, s2), {}),
            "config3": ((c2, s2), dict(stride=2, submanifold=False)),
            "config4": ((c3, ns3), dict(stride=2, transposed=True, submanifold=False)),
            "config5": (workloads.config5(seed=0), {})}


@pytest.mark.parametrize("name", sorted(LEDGER))
def test_ledger_on_benchmark_sets(sets, name):
    (c, shape), geom = sets[name]
    led = O.ledger(c, shape, kernel_size=3, padding=1, **geom)
    dropped, lost, entries, missing, false, wrong = LEDGER[name]
    assert led["insert_dropped"] == dropped
    assert led["entries"] == entries
    assert (led["missing"], led["false"], led["wrong"]) == (missing, false, wrong), led
    if lost is not None:
        assert led["outputs_lost"] == lost and led["outputs_spurious"] == 0
        assert led["same_order_as_first_occurrence"]  # one-at-a-time resolution keeps first occurrences
