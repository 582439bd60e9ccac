"""The device LRU's algorithm, pinned on the CPU against the reference-semantics
LRU (oracle.pool_oracle.LruSlots, a restatement of expert_pool.py:123-159).

``StampModel`` runs the steps of the device LRU (lru_assign in vm_lru.h) on numpy
arrays: distinct ids in first-seen order, hits stamped in that order, then the
misses take the non-hit slots with the smallest stamps, oldest first.  It must
hand out exactly the slots the OrderedDict LRU hands out, from a fresh pool and
from any host state converted with ``stamp_state`` (also after invalidations,
which reorder the free list).  No GPU needed.
"""
import random

import numpy as np

from oracle import pool_oracle
from veymoe.layout import RecordLayout
from veymoe.pool import ExpertPool, restore_from_stamps, stamp_state

LAYERS, EXPERTS = 6, 48


class StampModel:
    """The device assign on the host: table [layers, experts], owner/stamp per slot."""

    def __init__(self, table, owner, stamp, last):
        self.table = table.copy()
        self.owner = owner.copy()
        self.stamp = stamp.astype(np.uint64).copy()
        self.last = int(last)
        self.hits = 0
        self.misses = 0

    def assign(self, layer, routed):
        distinct = list(dict.fromkeys(int(e) for e in routed))
        row = self.table[layer]
        hit_slots = [int(row[e]) for e in distinct if row[e] >= 0]
        missed = [e for e in distinct if row[e] < 0]
        base = self.last
        for i, slot in enumerate(hit_slots):
            self.stamp[slot] = base + 1 + i
        slots = {e: int(row[e]) for e in distinct if row[e] >= 0}
        misses = []
        if missed:
            candidates = np.flatnonzero(self.stamp > 0)
            order = candidates[np.argsort(self.stamp[candidates], kind="stable")]
            victims = [int(s) for s in order if s not in set(hit_slots)][:len(missed)]
            assert len(victims) == len(missed)
            for m, (expert, slot) in enumerate(zip(missed, victims)):
                old = int(self.owner[slot])
                if old >= 0:
                    self.table[old // EXPERTS, old % EXPERTS] = -1
                self.owner[slot] = layer * EXPERTS + expert
                self.table[layer, expert] = slot
                self.stamp[slot] = base + 1 + len(hit_slots) + m
                slots[expert] = slot
                misses.append((expert, slot))
        self.last = base + len(hit_slots) + len(missed)
        self.hits += len(hit_slots)
        self.misses += len(missed)
        return slots, misses


def _pool(slots):
    return ExpertPool(RecordLayout(256, 128), slots, layers=LAYERS, experts=EXPERTS, device="cpu")


def _model_of(pool):
    owner, stamp, last = stamp_state(pool)
    return StampModel(pool._host_table, owner, stamp, last)


def _random_calls(rnd, count, tokens_max=3, top_k=5):
    for _ in range(count):
        layer = rnd.randrange(LAYERS)
        routed = []
        for _t in range(rnd.randrange(1, tokens_max + 1)):
            routed += rnd.sample(range(EXPERTS), top_k)   # one token: distinct experts in rank order
        yield layer, routed


def test_stamp_model_equals_the_reference_lru_from_a_fresh_pool():
    ref = pool_oracle.LruSlots(32)
    model = _model_of(_pool(32))
    rnd = random.Random(11)
    for layer, routed in _random_calls(rnd, 500):
        assert model.assign(layer, routed) == ref.assign(layer, routed)
    assert (model.hits, model.misses) == (ref.hits, ref.misses)
    for (layer, expert), slot in ref.slot_of.items():
        assert model.table[layer, expert] == slot
    assert (model.table >= 0).sum() == len(ref.slot_of)


def test_stamp_model_continues_a_warm_host_state_with_invalidations():
    pool = _pool(64)
    ref = pool_oracle.LruSlots(64)
    rnd = random.Random(5)
    for layer, routed in _random_calls(rnd, 6):
        got = pool.assign(layer, routed)
        assert got == ref.assign(layer, routed)
        if got[1]:
            pool.invalidate(layer, got[1][:2])
            ref.invalidate(layer, got[1][:2])
    fresh = [e for e in range(EXPERTS) if not pool.resident(5, e)][:5]
    got = pool.assign(5, fresh)
    assert got == ref.assign(5, fresh) and len(got[1]) == 5
    for lru in (pool, ref):
        lru.invalidate(5, [got[1][0], got[1][2]])   # free list ends low, high: pops high first
    assert pool._free == ref.free and pool._free != sorted(pool._free, reverse=True)  # reordered free list
    model = _model_of(pool)
    for layer, routed in _random_calls(rnd, 300):
        assert model.assign(layer, routed) == ref.assign(layer, routed)


def test_stamp_state_round_trips_the_host_lru():
    pool = _pool(20)
    rnd = random.Random(9)
    for layer, routed in _random_calls(rnd, 60):
        _, misses = pool.assign(layer, routed)
        if rnd.random() < 0.3 and misses:
            pool.invalidate(layer, misses[:1])
    owner, stamp, last = stamp_state(pool)
    assert len(set(stamp[stamp > 0].tolist())) == int((stamp > 0).sum()) == pool.usable_slots
    assert last == pool.usable_slots
    before = (list(pool._slot_of.items()), list(pool._free), pool._host_table.copy())
    copy = _pool(20)
    restore_from_stamps(copy, owner, stamp)
    assert list(copy._slot_of.items()) == before[0]
    assert copy._free == before[1]
    np.testing.assert_array_equal(copy._host_table, before[2])
    # the restored pool continues exactly like the original
    for layer, routed in _random_calls(rnd, 100):
        assert copy.assign(layer, routed) == pool.assign(layer, routed)


def test_stamp_model_with_repeated_experts_across_tokens():
    """Tokens of one call that share experts: the distinct set is first-seen
    over tokens in order, the routed-hit count is positions minus misses."""
    ref = pool_oracle.LruSlots(16)
    model = _model_of(_pool(16))
    routed = [3, 1, 4, 1, 5, 9, 3, 2]
    got = model.assign(0, routed)
    assert got == ref.assign(0, routed)
    assert [e for e, _ in got[1]] == [3, 1, 4, 5, 9, 2]
    assert len(routed) - len(got[1]) == 2
