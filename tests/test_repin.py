"""Online repin selection (crates/model/src/moe.rs:1450-1508) through the
host-only entry styx_repin_select, which is the choice styx_moe_* applies
every repin_interval tokens.  No GPU.

Pinned by hand-worked cases (the 2x hysteresis with its max(hits, 1) floor,
the repin_max throttle, the stop at the first unprofitable pair) and by
properties on random hit counts that any correct selection has: swaps pair
the i-th coldest resident with the i-th hottest outsider, each passes the
2x test, and the first pair not taken fails it (or repin_max / a list ran
out)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from styx_amd._lib import load


def select(hits, slot_experts, repin_max):
    hits = np.ascontiguousarray(hits, np.uint64)
    se = np.ascontiguousarray(slot_experts, np.uint32)
    cap = max(repin_max, 1)
    ss, sx = np.zeros(cap, np.uint32), np.zeros(cap, np.uint32)
    n = C.c_int(-1)
    rc = load().styx_repin_select(hits.ctypes.data, len(hits), se.ctypes.data if len(se) else None,
                                  len(se), repin_max, ss.ctypes.data, sx.ctypes.data, C.byref(n))
    if rc:
        raise ValueError(load().styx_last_error().decode())
    return list(zip(ss[:n.value].tolist(), sx[:n.value].tolist()))


def test_worked_example():
    # residents e0 (5 hits, slot 0), e1 (1, slot 1), e2 (3, slot 2);
    # outsiders e3 10, e4 2, e5 1, e6 0
    hits = [5, 1, 3, 10, 2, 1, 0]
    # pair 0: e3 (10) vs coldest resident e1 (1): 10 >= 2 -> swap into slot 1
    # pair 1: e4 (2) vs e2 (3): 2 < 6 -> stop
    assert select(hits, [0, 1, 2], 2) == [(1, 3)]
    assert select(hits, [0, 1, 2], 0) == []


def test_hysteresis_floor_of_one_hit():
    # a resident with 0 hits is displaced only by an outsider with >= 2
    assert select([0, 1], [0], 2) == []
    assert select([0, 2], [0], 2) == [(0, 1)]
    # exactly twice the resident's hits is enough, one less is not
    assert select([3, 6], [0], 2) == [(0, 1)]
    assert select([3, 5], [0], 2) == []


def test_repin_max_throttles():
    E = 16
    hits = np.zeros(E, np.uint64)
    hits[8:] = 100  # every outsider is hot, every resident cold
    slots = list(range(8))
    assert len(select(hits, slots, 2)) == 2
    assert len(select(hits, slots, 5)) == 5
    assert len(select(hits, slots, 100)) == 8   # bounded by the residents


def test_ties_keep_list_order():
    # equal hits: residents in slot order, outsiders in expert order
    hits = [0, 0, 0, 4, 4, 4]
    assert select(hits, [2, 0, 1], 3) == [(0, 3), (1, 4), (2, 5)]


def test_stops_at_first_unprofitable_pair():
    # pair 1 fails (4 < 2*3) and ends the selection, as the reference's
    # break: down the ranked lists residents only get hotter and outsiders
    # colder, so no later pair can pass
    hits = [1, 3, 9, 10, 4, 0]
    assert select(hits, [0, 1, 2], 3) == [(0, 3)]


@pytest.mark.parametrize("seed", range(20))
def test_properties_random(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.choice([16, 64, 128]))
    n_slots = int(rng.integers(0, E + 1))
    hits = rng.integers(0, 50, E).astype(np.uint64) * rng.integers(0, 2, E).astype(np.uint64)
    slots = rng.permutation(E)[:n_slots].astype(np.uint32)
    rmax = int(rng.integers(0, 6))
    sw = select(hits, slots, rmax)
    resident = set(slots.tolist())
    res_rank = sorted(range(n_slots), key=lambda s: (int(hits[slots[s]]), s))
    out_rank = sorted((e for e in range(E) if e not in resident), key=lambda e: (-int(hits[e]), e))
    assert len(sw) <= rmax
    for i, (slot, e) in enumerate(sw):
        assert slot == res_rank[i] and e == out_rank[i]
        assert hits[e] >= 2 * max(int(hits[slots[slot]]), 1)
    i = len(sw)
    if i < rmax and i < n_slots and i < len(out_rank):
        assert hits[out_rank[i]] < 2 * max(int(hits[slots[res_rank[i]]]), 1)


def test_rejects_bad_slot_lists():
    with pytest.raises(ValueError):
        select([1, 2, 3], [0, 0], 2)      # duplicate resident
    with pytest.raises(ValueError):
        select([1, 2, 3], [5], 2)         # id past n_expert
