"""CPU tests of the device prefix store and the slot-addressed pass table.

The store must keep PrefixCache's semantics (crates/cev-model/src/engine.rs:
474-503): the Python restatement below follows that code line for line and
the store's entry order is compared with it after every operation of random
request streams.  The slot table must give every pass row exactly the keys
the reference's dense mask (engine.rs:418-442) gives it, with the mask's
columns (plans' pasts concatenated in plan order, then the pass tokens)
mapped to the cache slots where the store keeps them."""
import numpy as np
import pytest

import cev_hip
from cev_hip._abi import CEV_ERR_INVALID, CEV_ERR_SPACE, CevError


class RefPrefixCache:
    """engine.rs:474-503: entries in LRU order, budget on total key length."""

    def __init__(self, budget):
        self.budget, self.entries = budget, []

    def get(self, key):
        for i, (k, _) in enumerate(self.entries):
            if k == key:
                e = self.entries.pop(i)
                self.entries.append(e)
                return e[1]
        return None

    def put(self, key, kv):
        if len(key) > self.budget:
            return
        self.entries = [e for e in self.entries if e[0] != key]
        self.entries.append((key, kv))
        while sum(len(k) for k, _ in self.entries) > self.budget:
            self.entries.pop(0)


def test_store_follows_prefix_cache_lru(cev):
    rng = np.random.default_rng(0)
    budget = 400
    store = cev_hip.PrefixStore(capacity=4096, budget=budget)
    ref = RefPrefixCache(budget)
    keys = [tuple(int(x) for x in rng.integers(0, 50, int(rng.integers(20, 160)))) for _ in range(12)]
    keys.append(tuple(range(500)))  # longer than the budget: never cached
    slot_of = {}
    for step in range(300):
        key = keys[int(rng.integers(len(keys)))]
        hit = store.get(key)
        want = ref.get(key)
        assert (hit is not None) == (want is not None), step
        if hit is None:
            b = store.reserve(len(key))
            store.put(key, b)
            ref.put(key, b)
            store.release(b)
            slot_of[key] = b
        else:
            assert hit == slot_of[key]
            store.release(hit)
        got = store.entries()
        assert [n for _, n in got] == [len(k) for k, _ in ref.entries]
        assert [b for b, _ in got] == [slot_of[k] for k, _ in ref.entries]
        st = store.stats()
        assert st["cached_tokens"] == sum(len(k) for k, _ in ref.entries) <= budget
        assert st["used_slots"] == st["cached_tokens"]  # nothing held between requests


def test_held_ranges_survive_eviction_and_free_on_release(cev):
    store = cev_hip.PrefixStore(capacity=100, budget=60)
    a = store.reserve(40)
    store.put(list(range(40)), a)          # held by its pass
    b = store.reserve(30)
    store.put(list(range(100, 130)), b)    # evicts a (70 > 60) ...
    assert store.entries() == [(b, 30)]
    assert store.stats()["used_slots"] == 70  # ... but a's pass still holds it
    c = None
    with pytest.raises(CevError) as e:
        c = store.reserve(40)              # only 30 free slots, every range held
    assert e.value.code == CEV_ERR_SPACE and c is None
    store.release(a)
    assert store.stats()["used_slots"] == 30
    store.release(b)
    # free runs [0, 40) and [70, 100): no 60 fit, so the unheld entry b goes
    c = store.reserve(60)
    assert c == 0 and store.entries() == []
    store.release(c)
    # a key longer than the budget is not cached, and its range frees on release
    d = store.reserve(70)
    store.put(list(range(70)), d)
    assert store.get(list(range(70))) is None
    store.release(d)
    with pytest.raises(CevError) as e:
        store.put(list(range(5)), 3)       # not a held reservation
    assert e.value.code == CEV_ERR_INVALID


def test_fragmented_store_evicts_oldest_unheld_entries(cev):
    store = cev_hip.PrefixStore(capacity=100, budget=100)
    rs = []
    for i in range(4):
        r = store.reserve(25)
        store.put([1000 * i + j for j in range(25)], r)
        store.release(r)
        rs.append(r)
    held = store.get([1000 + j for j in range(25)])  # entry 1 held by a pass (now newest)
    # no free run of 40: the oldest unheld entries go one by one until one
    # fits: entry 0 and entry 2 leave two 25-slot holes around the held
    # entry 1, entry 3 then frees [50, 100)
    big = store.reserve(40)
    assert store.entries() == [(rs[1], 25)]
    assert big == 50
    store.release(big)
    store.release(held)


def _slot_layout(rng, plans_spec, items_spec, capacity):
    """Non-overlapping slot ranges for every plan's prefix and question."""
    sizes = [p[1] for p in plans_spec] + [i[1] for i in items_spec]
    order = rng.permutation(len(sizes))
    gaps = rng.integers(0, 5, len(sizes))
    starts = np.zeros(len(sizes), np.int64)
    pos = 0
    for j in order:
        pos += int(gaps[j])
        starts[j] = pos
        pos += sizes[j]
    assert pos <= capacity
    kv_begin = [int(starts[i]) for i in range(len(plans_spec))]
    item_slot = [int(starts[len(plans_spec) + k]) for k in range(len(items_spec))]
    return kv_begin, item_slot


def test_slot_table_sees_exactly_the_engine_mask(cev, orc):
    rng = np.random.default_rng(4)
    for case in range(60):
        n_plans = int(rng.integers(1, 4))
        plans = []
        for _ in range(n_plans):
            pre = int(rng.integers(0, 90))
            ts = int(rng.integers(0, pre + 1))
            plans.append((ts, pre, ts))  # past = the computed head
        items = [(int(rng.integers(n_plans)), int(rng.integers(1, 30))) for _ in range(int(rng.integers(0, 6)))]
        if all(p[1] == p[2] for p in plans) and not items:
            continue
        capacity = 600
        kv_begin, item_slot = _slot_layout(rng, plans, items, capacity)
        tab, pos, slots, gather = cev_hip.BlockTable.from_slots([(kv_begin[p], pl[1], pl[2]) for p, pl in enumerate(plans)],
                                                                [(i[0], i[1], item_slot[k]) for k, i in enumerate(items)], capacity)
        ep = orc.engine_pass(plans, items)
        assert np.array_equal(pos, ep["pos"]) and np.array_equal(gather, ep["gather"])
        dense = tab.to_dense_mask()  # (t, capacity + t) over slot keys
        # reference column -> slot: plan p's past column j is slot kv_begin[p] + j
        col_slot = []
        for p, pl in enumerate(plans):
            col_slot += [kv_begin[p] + j for j in range(pl[0])]
        col_slot += list(slots)
        got = dense[:, col_slot]
        assert np.array_equal(got, ep["mask"]), case
        # and nothing else is visible
        others = np.ones(capacity + ep["n"], bool)
        others[col_slot] = False
        assert np.isneginf(dense[:, others]).all(), case


def test_slot_table_rejects_overlapping_writes(cev):
    with pytest.raises(CevError):   # question slots inside a plan's computed past
        cev_hip.BlockTable.from_slots([(0, 50, 50)], [(0, 10, 40)], 200)
    with pytest.raises(CevError):   # two questions on the same slots
        cev_hip.BlockTable.from_slots([(0, 50, 50)], [(0, 10, 60), (0, 10, 65)], 200)
    with pytest.raises(CevError):   # a tail written over another plan's past
        cev_hip.BlockTable.from_slots([(0, 50, 20), (30, 40, 40)], [], 200)
    with pytest.raises(CevError):   # beyond the capacity
        cev_hip.BlockTable.from_slots([(0, 50, 50)], [(0, 10, 195)], 200)
    # two plans reading the same cached prefix is fine
    tab, _, _, _ = cev_hip.BlockTable.from_slots([(0, 50, 50), (0, 50, 50)], [(0, 4, 60), (1, 4, 70)], 200)
    assert len(tab) == 2
