"""Record layout and expert-pool slot table (host side, no GPU)."""
import random

import numpy as np
import pytest
import torch

from oracle import pool_oracle
from veymoe.layout import HEADER, PARTS, RecordLayout, pack_record, unpack_record
from veymoe.pool import ExpertPool, HostRecordStore


def test_reference_slab_constants():
    # models/flashnext/tests/unit/test_slab_pack.py:50-63 (hidden 2560, inter 640)
    layout = RecordLayout(2560, 640)
    assert layout.record_stride == 3_072_000 and layout.record_stride % 4096 == 0
    expected = [0, 819_200, 921_600, 1_024_000, 1_843_200, 1_945_600, 2_048_000, 2_867_200, 2_969_600]
    assert layout.part_offsets() == expected
    assert layout.offset("down_proj", "biases") + 102_400 == layout.record_stride
    assert HEADER == 4096


@pytest.mark.parametrize("hidden,inter,stride", [(2048, 512, 1_966_080), (1024, 256, 491_520), (2560, 640, 3_072_000)])
def test_generalised_layout_matches_restatement(hidden, inter, stride):
    layout = RecordLayout(hidden, inter)
    offsets, sizes, ostride = pool_oracle.record_layout(hidden, inter)
    assert layout.record_stride == ostride == stride
    assert layout.record_bytes == int(1.875 * hidden * inter)
    for key in PARTS:
        assert layout.offset(*key) == offsets[key]
        assert layout.sizes[key] == sizes[key]
        assert layout.offset(*key) % 16 == 0


def test_pack_unpack_round_trip():
    layout = RecordLayout(256, 128)
    rng = np.random.default_rng(2)
    parts = {key: (rng.integers(0, 2 ** 32, size=layout.shape(*key), dtype=np.uint32) if key[1] == "weight"
                   else rng.integers(0, 2 ** 16, size=layout.shape(*key), dtype=np.uint16)) for key in PARTS}
    record = pack_record(parts, layout)
    back = unpack_record(record, layout)
    for key in PARTS:
        np.testing.assert_array_equal(back[key], parts[key])
    with pytest.raises(ValueError):
        bad = dict(parts)
        bad[("gate_proj", "weight")] = parts[("gate_proj", "weight")][:, :-1]
        pack_record(bad, layout)


def _pools(slots):
    layout = RecordLayout(256, 128)
    return ExpertPool(layout, slots, layers=8, experts=64, device="cpu"), pool_oracle.LruSlots(slots)


def test_hits_misses_and_lru_eviction():
    # models/flashnext/tests/unit/test_expert_pool.py:51-68
    for pool in _pools(16):
        slots, misses = pool.assign(1, list(range(10)))
        assert len(misses) == 10 and len(set(slots.values())) == 10
        slots2, misses2 = pool.assign(1, [3, 4, 20])
        assert slots2[3] == slots[3]
        assert [e for e, _ in misses2] == [20]
        pool.assign(2, list(range(5)))
        slots3, misses3 = pool.assign(1, [3, 4, 30, 31])
        assert slots3[3] == slots[3] and slots3[4] == slots[4]
        assert {slot for _, slot in misses3} == {slots[0], slots[1]}
        assert pool.hits == 2 + 2
        assert pool.misses == 10 + 1 + 5 + 2


def test_too_small_pool_is_refused():
    with pytest.raises(ValueError):
        ExpertPool(RecordLayout(256, 128), 4, device="cpu")
    with pytest.raises(ValueError):
        pool_oracle.LruSlots(4)


def test_oversized_assignment_fails_before_mutation():
    # test_expert_pool.py:74-80
    pool, _ = _pools(16)
    pool.assign(1, [1, 2, 3])
    before = (list(pool._slot_of.items()), list(pool._free), pool.hits, pool.misses, pool._host_table.copy())
    with pytest.raises(ValueError, match="exceed"):
        pool.assign(1, list(range(17)))
    after = (list(pool._slot_of.items()), list(pool._free), pool.hits, pool.misses, pool._host_table.copy())
    assert before[:4] == after[:4]
    np.testing.assert_array_equal(before[4], after[4])


def test_pool_matches_restatement_on_a_random_sequence():
    pool, ref = _pools(40)
    rnd = random.Random(4)
    for _ in range(400):
        layer = rnd.randrange(8)
        experts = [rnd.randrange(64) for _ in range(rnd.randrange(1, 12))]
        got = pool.assign(layer, experts)
        want = ref.assign(layer, experts)
        assert got == want
        if rnd.random() < 0.05 and got[1]:
            pool.invalidate(layer, got[1])
            ref.invalidate(layer, got[1])
        assert list(pool._slot_of.items()) == list(ref.slot_of.items())
        assert pool._free == ref.free
    # the device slot table mirror agrees with the LRU map
    table = np.full((8, 64), -1, np.int32)
    for (layer, expert), slot in pool._slot_of.items():
        table[layer, expert] = slot
    np.testing.assert_array_equal(pool._host_table, table)


def test_invalidate_returns_slots_and_never_hits():
    pool, _ = _pools(16)
    pool.assign(4, [1])
    _, misses = pool.assign(4, [2])
    pool.invalidate(4, misses)
    assert (4, 1) in pool._slot_of and (4, 2) not in pool._slot_of
    assert pool._host_table[4, 2] == -1
    _, retry = pool.assign(4, [2])
    assert [e for e, _ in retry] == [2]


def test_failed_fill_invalidates_misses():
    """A fill that cannot find its source rows leaves no partial record mapped
    (expert_cache.py:1895-1906, expert_pool.py:222-231)."""
    pool, _ = _pools(16)
    store = HostRecordStore(pool.layout, 4, pin=False)
    store.put(0, 1, np.zeros(pool.layout.record_stride, np.uint8))
    pool.assign(0, [1])
    _, misses = pool.assign(0, [7])
    with pytest.raises(KeyError):
        pool.fill(0, misses, store)
    assert (0, 7) not in pool._slot_of and (0, 1) in pool._slot_of


def test_place_and_from_bytes():
    layout = RecordLayout(2048, 512)
    pool = ExpertPool.from_bytes(layout, HEADER + 20 * layout.record_stride + 100, device="cpu", experts=512)
    assert pool.slots == 20
    pool.place(0, 5, 3)
    assert pool._host_table[0, 5] == 3 and 3 not in pool._free
    with pytest.raises(ValueError):
        pool.place(0, 6, 3)
    # reference slot count at 6 GB (expert_pool.py:92)
    assert (6_000_000_000 - HEADER) // layout.record_stride == 3051


def test_host_record_store_rows():
    layout = RecordLayout(256, 128)
    store = HostRecordStore(layout, 3, pin=False)
    rec = np.arange(layout.record_stride, dtype=np.uint64).astype(np.uint8)
    row = store.put(2, 9, rec)
    assert store.row(2, 9) == row == 0
    np.testing.assert_array_equal(store.buffer[0].numpy(), rec)
    store.alias(3, 9, row)
    assert store.row(3, 9) == 0
    with pytest.raises(KeyError):
        store.row(1, 1)
    assert isinstance(store.buffer, torch.Tensor)
