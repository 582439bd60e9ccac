"""HBM-resident expert pool with an LRU slot table.

Counterpart of the reference's ``ExpertPool`` (models/flashnext/expert_pool.py:78-294):

* one device allocation: a 4 KiB header, then fixed-stride expert records
  (``veymoe.layout.RecordLayout``), addressed by the kernels through route
  words ``SLOT_BIT | slot`` or through a per-layer int32 slot table
  (expert -> slot, -1 = absent) that the kernels read on the device;
* ``assign`` has the reference's LRU semantics exactly (expert_pool.py:123-159):
  distinct experts in first-seen order, hits move to the most recent end and
  are counted once per distinct expert, misses take the lowest free slot or
  evict the least recently used key, and a distinct set larger than the pool is
  refused before any state changes;
* misses are filled from pinned host memory (``HostRecordStore``, standing in
  for the SSD reads of ``fill``/``_fill_part``, :201-220, :258-287) with
  ``hipMemcpyAsync`` on a side stream (``vm_pool_stage``); an event joins the
  compute stream, and the copy stream first waits for the compute stream so a
  slot is overwritten only after its last reader (:19-22);
* a failed fill invalidates its misses so no partial record becomes a hit
  (``invalidate``, :222-231);
* ``attach_device_lru`` moves the LRU state to the device (``DeviceLru``):
  decode layers then assign, fill and run with ``vm_moe_layer_lru`` without
  any route sync to the host (the reference syncs every layer,
  expert_cache.py:1738-1749).  Recency there is one queue of slot ids (the
  free list in pop order, then the OrderedDict's slots), converted from and
  back to this class's state exactly.
"""
from __future__ import annotations

import ctypes
from collections import OrderedDict
from typing import Iterable

import numpy as np
import torch

from . import _lib
from .device import stream_handle
from .layout import HEADER, PARTS, SLOT_BIT, RecordLayout


class HostRecordStore:
    """Expert records in pinned host memory, keyed by (layer, expert)."""

    def __init__(self, layout: RecordLayout, capacity: int, pin: bool = True):
        self.layout = layout
        self.capacity = int(capacity)
        self.buffer = torch.empty((self.capacity, layout.record_stride), dtype=torch.uint8, pin_memory=pin)
        self._row_of = {}

    def __contains__(self, key):
        return key in self._row_of

    def put(self, layer: int, expert: int, record: np.ndarray) -> int:
        key = (int(layer), int(expert))
        row = self._row_of.get(key)
        if row is None:
            row = len(self._row_of)
            if row >= self.capacity:
                raise ValueError("host record store is full")
            self._row_of[key] = row
        self.buffer[row].numpy()[: record.size] = record
        return row

    def alias(self, layer: int, expert: int, row: int) -> None:
        """Map (layer, expert) to an existing row (records shared between ids)."""
        if not 0 <= row < self.capacity:
            raise ValueError("row outside the store")
        self._row_of[(int(layer), int(expert))] = int(row)

    def row(self, layer: int, expert: int) -> int:
        return self._row_of[(int(layer), int(expert))]


class ExpertPool:
    def __init__(self, layout: RecordLayout, slots: int, *, layers: int = 1, experts: int = 512,
                 device=None, header_size: int = HEADER):
        if slots < 16:
            raise ValueError("expert pool is too small for one decode layer")
        self.layout = layout
        self.slots = int(slots)
        self.layers = int(layers)
        self.experts = int(experts)
        self.header_size = int(header_size)
        self.stride = layout.record_stride
        self.device = torch.device("cuda") if device is None else torch.device(device)
        self.buffer = torch.zeros(self.header_size + self.slots * self.stride, dtype=torch.uint8,
                                  device=self.device)
        self.slot_table = torch.full((self.layers, self.experts), -1, dtype=torch.int32, device=self.device)
        self._host_table = np.full((self.layers, self.experts), -1, dtype=np.int32)
        self._dirty = set()
        self._slot_of: "OrderedDict[tuple, int]" = OrderedDict()
        self._free = list(range(self.slots - 1, -1, -1))
        self.hits = 0
        self.misses = 0
        self.bytes_staged = 0
        self._copy_stream = None
        self._pinned_table = None
        self._row_events = {}      # layer -> event after the last upload of its pinned row
        self._stage_events = None  # (compute reached the copies, copies done), reused
        self._stage_args = None    # ctypes index arrays, grown on demand
        self.device_lru = None     # DeviceLru while the LRU state lives on the device

    @classmethod
    def from_bytes(cls, layout: RecordLayout, size_bytes: int, **kwargs):
        """Size the pool like the reference: (bytes - header) // stride slots (expert_pool.py:92)."""
        header = kwargs.get("header_size", HEADER)
        return cls(layout, (int(size_bytes) - header) // layout.record_stride, **kwargs)

    # ------------------------------------------------------------ LRU ---
    @property
    def usable_slots(self) -> int:
        return len(self._free) + len(self._slot_of)

    def _map(self, key, slot):
        layer, expert = key
        self._host_table[layer, expert] = slot
        self._dirty.add(layer)

    def _unmap(self, key):
        layer, expert = key
        self._host_table[layer, expert] = -1
        self._dirty.add(layer)

    def _host_state(self, what: str) -> None:
        if self.device_lru is not None:
            raise RuntimeError(f"{what}: the LRU of this pool lives on the device (detach_device_lru first)")

    def assign(self, layer: int, experts: Iterable[int] | int):
        """Assign a distinct expert set that fits in the pool, or fail before mutation."""
        self._host_state("assign")
        if isinstance(experts, (int, np.integer)):
            experts = [int(experts)]
        distinct = list(dict.fromkeys(int(e) for e in experts))
        if len(distinct) > self.usable_slots:
            raise ValueError("requested experts exceed expert pool capacity")
        slot_of = self._slot_of
        slots, misses = {}, []
        for expert in distinct:
            slot = slot_of.get((layer, expert))
            if slot is not None:
                slot_of.move_to_end((layer, expert))
                slots[expert] = slot
        self.hits += len(slots)
        for expert in distinct:
            if expert in slots:
                continue
            if self._free:
                slot = self._free.pop()
            else:
                old, slot = slot_of.popitem(last=False)
                self._unmap(old)
            slot_of[(layer, expert)] = slot
            self._map((layer, expert), slot)
            slots[expert] = slot
            misses.append((expert, slot))
        self.misses += len(misses)
        return slots, misses

    def invalidate(self, layer: int, misses) -> None:
        """Return the slots of failed fills to the free list, never as hits."""
        self._host_state("invalidate")
        for expert, slot in misses:
            key = (layer, expert)
            if self._slot_of.get(key) == slot:
                self._free.append(self.discard_slot(key))

    def discard_slot(self, key):
        slot = self._slot_of.pop(key)
        self._unmap(key)
        return slot

    def resident(self, layer: int, expert: int) -> bool:
        return (layer, expert) in self._slot_of

    def holds_every_key(self) -> bool:
        """Every (layer, expert) of the pool's table is mapped: no assign can
        miss, so none evicts.  Mappings written straight into the host table
        (static setups that share records between experts) count as well."""
        return len(self._slot_of) == self.layers * self.experts or bool((self._host_table >= 0).all())

    # ---------------------------------------------------------- device ---
    def view(self) -> _lib.VmPoolView:
        view = _lib.VmPoolView()
        view.base = self.buffer.data_ptr()
        view.header_size = self.header_size
        view.record_stride = self.stride
        for i, offset in enumerate(self.layout.part_offsets()):
            view.part_offset[i] = offset
        view.records = self.slots
        return view

    def table(self, layer: int) -> torch.Tensor:
        return self.slot_table[layer]

    def sync_tables(self) -> None:
        """Upload the slot-table rows changed since the last call, asynchronously
        on the current stream (ordered before any kernel launched after it),
        from a pinned mirror row that is rewritten only after its last upload
        ran (one event per row, normally complete by then)."""
        if not self._dirty:
            return
        if self._pinned_table is None:
            self._pinned_table = torch.empty((self.layers, self.experts), dtype=torch.int32,
                                             pin_memory=self.device.type == "cuda")
        stream = torch.cuda.current_stream(self.device)
        for layer in sorted(self._dirty):
            event = self._row_events.get(layer)
            if event is None:
                event = self._row_events[layer] = torch.cuda.Event()
            elif not event.query():
                event.synchronize()
            self._pinned_table[layer].numpy()[:] = self._host_table[layer]
            self.slot_table[layer].copy_(self._pinned_table[layer], non_blocking=True)
            event.record(stream)
        self._dirty.clear()

    def place(self, layer: int, expert: int, slot: int) -> None:
        """Pin (layer, expert) to ``slot`` directly (resident setups); the slot
        must be free."""
        self._host_state("place")
        key = (int(layer), int(expert))
        if key in self._slot_of:
            raise ValueError(f"{key} is already resident")
        try:
            self._free.remove(int(slot))
        except ValueError:
            raise ValueError(f"slot {slot} is not free") from None
        self._slot_of[key] = int(slot)
        self._map(key, int(slot))

    def place_all(self, layer: int, slots) -> None:
        """Pin expert e of ``layer`` to ``slots[e]`` for every e (resident setups)."""
        self._host_state("place_all")
        slots = [int(s) for s in slots]
        taken = set(slots)
        if len(taken) != len(slots) or not taken.issubset(self._free):
            raise ValueError("slots must be distinct and free")
        for expert, slot in enumerate(slots):
            key = (int(layer), expert)
            if key in self._slot_of:
                raise ValueError(f"{key} is already resident")
            self._slot_of[key] = slot
            self._map(key, slot)
        self._free = [s for s in self._free if s not in taken]

    def record(self, slot: int) -> torch.Tensor:
        """Device bytes of one record (a view)."""
        start = self.header_size + int(slot) * self.stride
        return self.buffer[start:start + self.stride]

    def copy_stream(self):
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(device=self.device)
        return self._copy_stream

    def stage(self, source: HostRecordStore, layer: int, misses, compute_stream=None) -> torch.cuda.Event | None:
        """Copy the records of ``misses`` [(expert, slot)] from pinned host memory
        into their slots on the side stream; the compute stream waits for it.
        Returns the completion event, which the next call records again."""
        if not misses:
            return None
        self._host_state("stage")
        order = sorted(misses, key=lambda item: item[1])
        n = len(order)
        if self._stage_args is None or len(self._stage_args[0]) < n:
            size = max(64, n)
            self._stage_args = ((ctypes.c_int64 * size)(), (ctypes.c_int64 * size)())
        src, dst = self._stage_args
        for i, (expert, slot) in enumerate(order):
            src[i] = source.row(layer, expert)
            dst[i] = slot
        compute = torch.cuda.current_stream(self.device) if compute_stream is None else compute_stream
        copier = self.copy_stream()
        if self._stage_events is None:
            self._stage_events = (torch.cuda.Event(), torch.cuda.Event())
        reached, done = self._stage_events
        # a slot may still be read by kernels queued before this point
        reached.record(compute)
        copier.wait_event(reached)
        rc = _lib.lib().vm_pool_stage(
            self.buffer.data_ptr(), self.header_size, self.stride, self.slots,
            source.buffer.data_ptr(), source.layout.record_stride, source.capacity,
            self.layout.record_bytes, src, dst, n, stream_handle(copier))
        if rc != _lib.VM_OK:
            self.invalidate(layer, misses)
            _lib.check(rc)
        done.record(copier)
        compute.wait_event(done)
        self.bytes_staged += n * self.layout.record_bytes
        return done

    def fill(self, layer: int, misses, source: HostRecordStore, compute_stream=None):
        """Stage misses; on any failure invalidate them before re-raising."""
        try:
            return self.stage(source, layer, misses, compute_stream)
        except BaseException:
            self.invalidate(layer, misses)
            raise


    # ------------------------------------------------------ device LRU ---
    def attach_device_lru(self, source: HostRecordStore, reuse: "DeviceLru" = None) -> "DeviceLru":
        """Move the LRU state to the device; misses are then filled from
        ``source`` by the GPU itself.  Host-side LRU calls raise until
        ``detach_device_lru``.  ``reuse``: a device LRU this pool detached
        earlier; its buffers take the current state, so step graphs recorded
        over them stay valid (a new one is made if the queue length changed)."""
        if self.device_lru is not None:
            raise RuntimeError("a device LRU is already attached")
        if reuse is not None and reuse.pool is self and reuse.store is source and reuse.reload():
            self.device_lru = reuse
        else:
            self.device_lru = DeviceLru(self, source)
        return self.device_lru

    def detach_device_lru(self) -> None:
        """Bring the LRU state back from the device (one sync)."""
        lru = self.device_lru
        if lru is None:
            return
        table, owner, order = lru.state()
        restore_from_order(self, owner, order)
        if not np.array_equal(table, self._host_table):
            raise RuntimeError("device slot table disagrees with the slot owners")
        stats = lru.stats()
        self.hits += stats["hits"]
        self.misses += stats["misses"]
        self.bytes_staged += stats["misses"] * self.layout.record_bytes
        self.device_lru = None


def order_state(pool: ExpertPool):
    """The pool's LRU state in the form the device LRU keeps: one queue of
    slot ids, least recently used first, which is the free list in the order
    it pops (from its end) followed by the resident slots from least to most
    recently used (the OrderedDict order).  Slots that are neither free nor
    resident are not queued and never handed out.  Returns (owner [slots]
    int32 = layer * experts + expert or -1, order [usable_slots] int32)."""
    owner = np.full(pool.slots, -1, dtype=np.int32)
    for (layer, expert), slot in pool._slot_of.items():
        owner[slot] = layer * pool.experts + expert
    order = np.array(list(reversed(pool._free)) + list(pool._slot_of.values()), dtype=np.int32)
    return owner, order


def restore_from_order(pool: ExpertPool, owner: np.ndarray, order: np.ndarray) -> None:
    """Inverse of ``order_state``: rebuild the free list, the OrderedDict and
    the host slot table of ``pool`` from per-slot owners and the queue."""
    owner = np.asarray(owner)
    order = [int(s) for s in np.asarray(order)]
    if len(set(order)) != len(order) or any(not 0 <= s < pool.slots for s in order):
        raise RuntimeError("the LRU queue does not list distinct slots of the pool")
    pool._free = [s for s in reversed(order) if owner[s] < 0]
    pool._slot_of = OrderedDict()
    pool._host_table[:] = -1
    for slot in order:
        if owner[slot] >= 0:
            layer, expert = divmod(int(owner[slot]), pool.experts)
            pool._slot_of[(layer, expert)] = slot
            pool._host_table[layer, expert] = slot
    pool._dirty.clear()


class DeviceLru:
    """The LRU state of an ``ExpertPool`` on the device (``VmDeviceLru``):
    the slot table (the pool's own device table), per-slot owners, the LRU
    queue, counters, and the host-store row of every (layer, expert)."""

    def __init__(self, pool: ExpertPool, source: HostRecordStore):
        if source.layout.record_bytes != pool.layout.record_bytes:
            raise ValueError("host store records do not match the pool layout")
        if not source.buffer.is_pinned():
            raise ValueError("the host store must be pinned memory")
        pool.sync_tables()
        owner, order = order_state(pool)
        dev = pool.device
        self.pool = pool
        self.store = source
        self.usable_slots = pool.usable_slots
        self.slot_owner = torch.from_numpy(owner).to(dev)
        self.order_len = len(order)
        self.lru_order = torch.from_numpy(order).to(dev)
        counters = np.zeros(4 + 4 * pool.layers, dtype=np.int64)
        self.counters = torch.from_numpy(counters).to(dev)
        host_row = np.full((pool.layers, pool.experts), -1, dtype=np.int32)
        for (layer, expert), row in source._row_of.items():
            if layer < pool.layers and expert < pool.experts:
                host_row[layer, expert] = row
        self.host_row = torch.from_numpy(host_row).to(dev)
        self._views = {}

    def reload(self) -> bool:
        """Upload the pool's host LRU state into these buffers (same device
        addresses) and zero the counters, whose counts the detach folded into
        the pool.  False when the queue length changed (a slot was discarded)."""
        pool = self.pool
        pool.sync_tables()
        owner, order = order_state(pool)
        if len(order) != self.order_len:
            return False
        self.slot_owner.copy_(torch.from_numpy(owner))
        self.lru_order.copy_(torch.from_numpy(order))
        self.counters.zero_()
        return True

    def view(self, layer: int) -> _lib.VmDeviceLru:
        v = self._views.get(layer)
        if v is None:
            v = _lib.VmDeviceLru()
            v.slot_table = self.pool.slot_table.data_ptr()
            v.slot_owner = self.slot_owner.data_ptr()
            v.lru_order = self.lru_order.data_ptr()
            v.counters = self.counters.data_ptr()
            v.host_row = self.host_row.data_ptr()
            v.host_store = self.store.buffer.data_ptr()
            v.host_stride = self.store.buffer.stride(0)
            v.host_records = self.store.capacity
            v.layers = self.pool.layers
            v.layer = int(layer)
            v.slots = self.pool.slots
            v.order_len = self.order_len
            self._views[layer] = v
        return v

    def stats(self, layer: int = None) -> dict:
        """Counters (synchronizes): pool-wide, or of one layer."""
        c = self.counters.cpu().numpy()
        if layer is None:
            return {"assigned": int(c[0]), "hits": int(c[1]), "misses": int(c[2]), "routed_hits": int(c[3])}
        r = c[4 + 4 * layer: 8 + 4 * layer]
        return {"hits": int(r[0]), "misses": int(r[1]), "routed_hits": int(r[2]), "routed": int(r[3])}

    def state(self):
        """(slot table [layers, experts], owners [slots], LRU queue [order_len]) on the host."""
        return (self.pool.slot_table.cpu().numpy(), self.slot_owner.cpu().numpy(), self.lru_order.cpu().numpy())


def route_words(slots_of: dict, routed) -> np.ndarray:
    """``SLOT_BIT | slot`` for every routed expert (expert_cache.py:1915-1917)."""
    return np.array([SLOT_BIT | slots_of[int(e)] for e in routed], dtype=np.uint32)


__all__ = ["DeviceLru", "ExpertPool", "HostRecordStore", "PARTS", "SLOT_BIT", "order_state", "restore_from_order",
           "route_words"]
