"""CPU oracle of the expert pool's slot table and record layout.

TEST INFRASTRUCTURE ONLY (see oracle/moe_oracle.py).

* ``LruSlots`` restates ``ExpertPool.assign`` / ``invalidate`` /
  ``usable_slots`` (models/flashnext/expert_pool.py:92-93,112,119-159,222-238)
  for the default LRU policy: hits move to the most recent end (counted once
  per distinct expert), misses take the lowest free slot (the free list is
  built high-to-low and popped from the end) or evict the least recently used
  key, and an oversized distinct set is refused before any mutation.
* ``record_layout`` restates ``_make_layout`` (models/flashnext/slab_pack.py:96-149)
  with the hidden/intermediate sizes as parameters instead of the hard-coded
  2560/640.  Pinned against the reference's constants
  (tests/test_slab_pack.py:50-63 of the reference: 819,200 / 921,600 /
  1,024,000 / ... / 3,072,000).
"""
from __future__ import annotations

from collections import OrderedDict

HEADER = 4096
SLOT_BIT = 0x80000000
PARTS = (
    ("gate_proj", "weight"), ("gate_proj", "scales"), ("gate_proj", "biases"),
    ("up_proj", "weight"), ("up_proj", "scales"), ("up_proj", "biases"),
    ("down_proj", "weight"), ("down_proj", "scales"), ("down_proj", "biases"),
)


def record_layout(hidden, inter, group_size=32, page=4096):
    """(offsets dict {(proj, part): byte offset}, part sizes, record stride)."""
    shapes = {"gate_proj": (inter, hidden), "up_proj": (inter, hidden), "down_proj": (hidden, inter)}
    offsets, sizes = {}, {}
    cursor = 0
    for proj, part in PARTS:
        rows, cols = shapes[proj]
        size = rows * cols // 2 if part == "weight" else rows * (cols // group_size) * 2
        offsets[(proj, part)] = cursor
        sizes[(proj, part)] = size
        cursor += size
    stride = -(-cursor // page) * page
    return offsets, sizes, stride


class LruSlots:
    def __init__(self, slots):
        if slots < 16:
            raise ValueError("expert pool is too small for one decode layer")
        self.slots = slots
        self.slot_of = OrderedDict()
        self.free = list(range(slots - 1, -1, -1))
        self.hits = 0
        self.misses = 0

    @property
    def usable_slots(self):
        return len(self.free) + len(self.slot_of)

    def assign(self, layer, experts):
        if isinstance(experts, int):
            experts = [experts]
        distinct = list(dict.fromkeys(experts))
        if len(distinct) > self.usable_slots:
            raise ValueError("requested experts exceed expert pool capacity")
        slots, misses = {}, []
        for expert in distinct:
            slot = self.slot_of.get((layer, expert))
            if slot is not None:
                self.slot_of.move_to_end((layer, expert))
                slots[expert] = slot
        self.hits += len(slots)
        for expert in distinct:
            if expert in slots:
                continue
            if self.free:
                slot = self.free.pop()
            else:
                _old, slot = self.slot_of.popitem(last=False)
            self.slot_of[(layer, expert)] = slot
            slots[expert] = slot
            misses.append((expert, slot))
        self.misses += len(misses)
        return slots, misses

    def invalidate(self, layer, misses):
        for expert, slot in misses:
            key = (layer, expert)
            if self.slot_of.get(key) == slot:
                self.free.append(self.slot_of.pop(key))
