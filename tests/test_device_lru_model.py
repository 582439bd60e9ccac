"""The device LRU's algorithm, pinned on the CPU against the reference-semantics
LRU (oracle.pool_oracle.LruSlots, a restatement of expert_pool.py:123-159).

``QueueModel`` runs the steps of the device assign (lru_assign in vm_lru.h) on
numpy arrays, with the kernel's block arithmetic: 1024 threads each holding a
contiguous run of the queue, per-thread counts packed as kept | hits << 16,
inclusive sums per 64-lane wave, wave totals, and each kept entry's new
position from its thread's exclusive prefix.  It must hand out exactly the
slots the OrderedDict LRU hands out, from a fresh pool and from any host state
converted with ``order_state`` (also after invalidations, which reorder the
free list), for pools smaller and larger than one entry per thread.  No GPU
needed.
"""
import random

import numpy as np
import pytest

from oracle import pool_oracle
from veymoe.layout import RecordLayout
from veymoe.pool import ExpertPool, order_state, restore_from_order

LAYERS, EXPERTS = 6, 48
THREADS, WAVE = 1024, 64


class QueueModel:
    """The device assign on the host: table [layers, experts], owner per slot, queue."""

    def __init__(self, table, owner, order, slots):
        self.table = table.copy()
        self.owner = owner.copy()
        self.order = np.asarray(order, dtype=np.int64).copy()
        self.slots = slots
        self.hits = 0
        self.misses = 0

    def _ranks(self, kept_flags, hit_flags):
        """Exclusive prefix count of the kept entries at the start of every
        thread's run, as the kernel forms it."""
        U = len(self.order)
        per = -(-U // THREADS)
        pad = THREADS * per - U
        keep = np.concatenate([kept_flags, np.zeros(pad, bool)]).reshape(THREADS, per).sum(1)
        hitq = np.concatenate([hit_flags, np.zeros(pad, bool)]).reshape(THREADS, per).sum(1)
        packed = (keep | (hitq << 16)).astype(np.int64)
        incl = np.cumsum(packed.reshape(-1, WAVE), axis=1)             # per wave
        wsum = incl[:, -1]
        before = np.concatenate([[0], np.cumsum(wsum)[:-1]])           # earlier waves
        total = int(wsum.sum())
        start = ((before[:, None] + incl - packed.reshape(-1, WAVE)) & 0xFFFF).reshape(-1)
        return per, start, total & 0xFFFF, total >> 16

    def assign(self, layer, routed):
        distinct = list(dict.fromkeys(int(e) for e in routed))
        row = self.table[layer]
        hit_slots = [int(row[e]) for e in distinct if 0 <= row[e] < self.slots]
        missed = [e for e in distinct if not 0 <= row[e] < self.slots]
        H, M = len(hit_slots), len(missed)
        hit_set = set(hit_slots)
        hit_flags = np.array([int(s) in hit_set for s in self.order], bool)
        per, start, NH, HQ = self._ranks(~hit_flags, hit_flags)
        assert HQ == H
        found = min(M, NH)
        kept = NH - found
        new = self.order.copy()
        victims = [None] * found
        for t in range(THREADS):
            lo = t * per
            rank = int(start[t])
            for i in range(lo, min(lo + per, len(self.order))):
                if hit_flags[i]:
                    continue
                if rank < found:
                    victims[rank] = (int(self.order[i]), int(self.owner[self.order[i]]))
                else:
                    new[rank - found] = self.order[i]
                rank += 1
        for h, s in enumerate(hit_slots):
            new[kept + h] = s
        slots = {e: int(row[e]) for e in distinct if 0 <= row[e] < self.slots}
        misses = []
        for m, (v, old) in enumerate(victims):
            e = missed[m]
            if old >= 0:
                self.table[old // EXPERTS, old % EXPERTS] = -1
            self.owner[v] = layer * EXPERTS + e
            self.table[layer, e] = v
            new[kept + H + m] = v
            slots[e] = v
            misses.append((e, v))
        assert sorted(new.tolist()) == sorted(self.order.tolist())    # a permutation
        self.order = new
        self.hits += H
        self.misses += M
        return slots, misses


def _pool(slots, layers=LAYERS):
    return ExpertPool(RecordLayout(256, 128), slots, layers=layers, experts=EXPERTS, device="cpu")


def _model_of(pool):
    owner, order = order_state(pool)
    return QueueModel(pool._host_table, owner, order, pool.slots)


def _random_calls(rnd, count, tokens_max=3, top_k=5, layers=LAYERS):
    for _ in range(count):
        layer = rnd.randrange(layers)
        routed = []
        for _t in range(rnd.randrange(1, tokens_max + 1)):
            routed += rnd.sample(range(EXPERTS), top_k)   # one token: distinct experts in rank order
        yield layer, routed


def test_queue_model_equals_the_reference_lru_from_a_fresh_pool():
    ref = pool_oracle.LruSlots(32)
    model = _model_of(_pool(32))
    rnd = random.Random(11)
    for layer, routed in _random_calls(rnd, 500):
        assert model.assign(layer, routed) == ref.assign(layer, routed)
    assert (model.hits, model.misses) == (ref.hits, ref.misses)
    for (layer, expert), slot in ref.slot_of.items():
        assert model.table[layer, expert] == slot
    assert (model.table >= 0).sum() == len(ref.slot_of)
    assert model.order.tolist() == list(reversed(ref.free)) + list(ref.slot_of.values())


@pytest.mark.parametrize("slots", [1500, 2100, 4096])
def test_queue_model_with_several_entries_per_thread(slots):
    """Queues longer than 1024 entries: every thread holds a run of 2..4."""
    layers = 64                               # 3072 keys: evictions below 3072 slots
    ref = pool_oracle.LruSlots(slots)
    model = _model_of(_pool(slots, layers))
    rnd = random.Random(slots)
    for layer, routed in _random_calls(rnd, 900, tokens_max=8, top_k=10, layers=layers):
        assert model.assign(layer, routed) == ref.assign(layer, routed)
    assert model.order.tolist() == list(reversed(ref.free)) + list(ref.slot_of.values())
    assert (model.hits, model.misses) == (ref.hits, ref.misses)
    if slots < layers * EXPERTS:
        assert not ref.free                   # evictions happened


def test_queue_model_continues_a_warm_host_state_with_invalidations():
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


def test_order_state_round_trips_the_host_lru():
    pool = _pool(20)
    rnd = random.Random(9)
    for layer, routed in _random_calls(rnd, 60):
        _, misses = pool.assign(layer, routed)
        if rnd.random() < 0.3 and misses:
            pool.invalidate(layer, misses[:1])
    owner, order = order_state(pool)
    assert len(order) == len(set(order.tolist())) == pool.usable_slots
    assert order.tolist() == list(reversed(pool._free)) + list(pool._slot_of.values())
    before = (list(pool._slot_of.items()), list(pool._free), pool._host_table.copy())
    copy = _pool(20)
    restore_from_order(copy, owner, order)
    assert list(copy._slot_of.items()) == before[0]
    assert copy._free == before[1]
    np.testing.assert_array_equal(copy._host_table, before[2])
    # the restored pool continues exactly like the original
    for layer, routed in _random_calls(rnd, 100):
        assert copy.assign(layer, routed) == pool.assign(layer, routed)


def test_restore_refuses_a_queue_that_is_not_a_set_of_pool_slots():
    pool = _pool(20)
    owner, order = order_state(pool)
    for bad in (np.concatenate([order[:-1], order[:1]]), np.concatenate([order[:-1], [20]])):
        with pytest.raises(RuntimeError):
            restore_from_order(_pool(20), owner, bad)


def test_queue_model_with_repeated_experts_across_tokens():
    """Tokens of one call that share experts: the distinct set is first-seen
    over tokens in order, the routed-hit count is positions minus misses."""
    ref = pool_oracle.LruSlots(16)
    model = _model_of(_pool(16))
    routed = [3, 1, 4, 1, 5, 9, 3, 2]
    got = model.assign(0, routed)
    assert got == ref.assign(0, routed)
    assert [e for e, _ in got[1]] == [3, 1, 4, 5, 9, 2]
    assert len(routed) - len(got[1]) == 2
