"""GPU parity of the device-resident LRU decode path (vm_moe_layer_lru).

Every call must give the same bits as the dense layer, leave the device slot
table equal to the reference-semantics LRU (oracle.pool_oracle.LruSlots fed the
same routed ids, expert_pool.py:123-159), and fill every missed record byte for
byte from the pinned host store."""
import numpy as np
import pytest
import torch

from gpu_util import pooled_stack
from oracle import pool_oracle
from veymoe import assemble, synth

pytestmark = pytest.mark.gpu

SEED = 77
SMALL = synth.LayerSpec("lru_small", 256, 128, 64, 4, 128, 1)
FULL = synth.LayerSpec("lru_full", 2048, 512, 64, 10, 512, 1)


def _setup(device, spec, layers, slots):
    return pooled_stack(device, spec, layers, slots, SEED)


def _expected_table(ref, layers, experts):
    table = np.full((layers, experts), -1, np.int32)
    for (layer, expert), slot in ref.slot_of.items():
        table[layer, expert] = slot
    return table


def _step(spec, pooled, dense, layer, tokens, stream, device):
    x = assemble.tokens_tensor(spec, SEED, device, tokens, stream=stream)
    a = pooled[layer](x[None])
    b = dense[layer](x[None])
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (layer, tokens, stream)
    return pooled[layer].last_inds.cpu().numpy().reshape(-1).tolist()


def _check_records(pool, store, ref):
    nbytes = pool.layout.record_bytes
    for (layer, expert), slot in ref.slot_of.items():
        got = pool.record(slot)[:nbytes].cpu()
        want = store.buffer[store.row(layer, expert)][:nbytes]
        assert torch.equal(got, want), (layer, expert, slot)


def test_device_lru_matches_dense_layers_and_the_reference_lru(device):
    layers, slots = 3, 40
    store, pool, pooled, dense = _setup(device, SMALL, layers, slots)
    ref = pool_oracle.LruSlots(slots)
    lru = pool.attach_device_lru(store)
    token_counts = [1, 1, 2, 8, 3, 1, 5, 1]
    for step in range(36):
        layer = (step * 5) % layers
        routed = _step(SMALL, pooled, dense, layer, token_counts[step % len(token_counts)], step, device)
        ref.assign(layer, routed)
        table, owner, _ = lru.state()
        np.testing.assert_array_equal(table, _expected_table(ref, layers, SMALL.experts), err_msg=f"step {step}")
        for (l, e), slot in ref.slot_of.items():
            assert owner[slot] == l * SMALL.experts + e
    stats = lru.stats()
    assert (stats["hits"], stats["misses"]) == (ref.hits, ref.misses)
    assert stats["misses"] > slots          # evictions happened
    per_layer = [lru.stats(l) for l in range(layers)]
    assert sum(s["misses"] for s in per_layer) == ref.misses
    assert sum(s["routed"] for s in per_layer) == sum(token_counts[s % len(token_counts)] for s in range(36)) * 4
    _check_records(pool, store, ref)


def test_device_lru_continues_a_warm_host_state_and_detaches(device):
    layers, slots = 2, 32
    store, pool, pooled, dense = _setup(device, SMALL, layers, slots)
    ref = pool_oracle.LruSlots(slots)
    # host LRU first (router, host assign, hipMemcpyAsync staging), with an
    # invalidation that reorders the free list
    for step in range(6):
        routed = _step(SMALL, pooled, dense, step % layers, 2, 100 + step, device)
        ref.assign(step % layers, routed)
    _, misses = pool.assign(1, [e for e in range(SMALL.experts) if not pool.resident(1, e)][:3])
    ref_misses = ref.assign(1, [e for e, _ in misses])[1]
    assert ref_misses == misses
    pool.fill(1, misses, store)
    pool.invalidate(1, [misses[0], misses[2]])
    ref.invalidate(1, [misses[0], misses[2]])
    lru = pool.attach_device_lru(store)
    with pytest.raises(RuntimeError):
        pool.assign(0, [1])
    for step in range(20):
        layer = step % layers
        routed = _step(SMALL, pooled, dense, layer, 1 + step % 4, 200 + step, device)
        ref.assign(layer, routed)
    np.testing.assert_array_equal(lru.state()[0], _expected_table(ref, layers, SMALL.experts))
    _check_records(pool, store, ref)
    pool.detach_device_lru()
    assert list(pool._slot_of.items()) == list(ref.slot_of.items())
    assert pool._free == ref.free
    # the host LRU carries on from the restored state
    for step in range(4):
        routed = _step(SMALL, pooled, dense, step % layers, 1, 300 + step, device)
        ref.assign(step % layers, routed)
        assert list(pool._slot_of.items()) == list(ref.slot_of.items())


def test_rows_above_the_decode_bound_hand_the_state_back(device):
    layers, slots = 1, 48
    store, pool, pooled, dense = _setup(device, SMALL, layers, slots)
    ref = pool_oracle.LruSlots(slots)
    pool.attach_device_lru(store)
    for step, tokens in enumerate([1, 12, 2]):
        routed = _step(SMALL, pooled, dense, 0, tokens, 400 + step, device)
        ref.assign(0, routed)
        assert pool.device_lru is not None
    table = pool.device_lru.state()[0]
    np.testing.assert_array_equal(table, _expected_table(ref, layers, SMALL.experts))


def test_full_size_records_through_the_device_lru(device):
    """hidden 2048 / inter 512 records (1,966,080 bytes each) copied by the fill
    kernel from pinned host memory; top-10 + shared expert."""
    layers, slots = 1, 24
    store, pool, pooled, dense = _setup(device, FULL, layers, slots)
    ref = pool_oracle.LruSlots(slots)
    lru = pool.attach_device_lru(store)
    for step in range(8):
        routed = _step(FULL, pooled, dense, 0, 1 + step % 2, 500 + step, device)
        ref.assign(0, routed)
    np.testing.assert_array_equal(lru.state()[0], _expected_table(ref, layers, FULL.experts))
    assert lru.stats()["misses"] == ref.misses > slots
    _check_records(pool, store, ref)


def test_device_lru_queue_longer_than_one_block(device):
    """1100 slots: every thread of the assign block holds a run of two queue
    entries.  The pool is warmed by the host LRU (all 1280 keys in a shuffled
    order, so the queue starts with evictions behind it), then the device
    continues; its queue must equal the reference's free list + OrderedDict."""
    import random

    layers, slots = 20, 1100
    store, pool, pooled, dense = _setup(device, SMALL, layers, slots)
    ref = pool_oracle.LruSlots(slots)
    rnd = random.Random(3)
    for layer in rnd.sample(range(layers), layers):
        experts = rnd.sample(range(SMALL.experts), SMALL.experts)
        _, misses = pool.assign(layer, experts)
        assert misses == ref.assign(layer, experts)[1]
        pool.fill(layer, misses, store)
    host_hits, host_misses = ref.hits, ref.misses
    lru = pool.attach_device_lru(store)
    assert lru.order_len == slots
    for step in range(40):
        layer = rnd.randrange(layers)
        routed = _step(SMALL, pooled, dense, layer, 1 + step % 8, 600 + step, device)
        ref.assign(layer, routed)
        if step % 10 == 9:
            table, owner, order = lru.state()
            np.testing.assert_array_equal(table, _expected_table(ref, layers, SMALL.experts), err_msg=f"step {step}")
            assert order.tolist() == list(reversed(ref.free)) + list(ref.slot_of.values()), step
    stats = lru.stats()
    assert (stats["hits"], stats["misses"]) == (ref.hits - host_hits, ref.misses - host_misses)
    _check_records(pool, store, ref)


def test_a_queue_with_a_foreign_slot_leaves_the_state_untouched(device):
    """An entry outside 0..slots-1 in the queue: the call sets status bit 16,
    maps and fills nothing, and leaves table, owners, queue and counters as
    they were (the layer's experts then see unmapped slots: status bit 1)."""
    from veymoe import _lib
    from veymoe.device import stream_handle

    layers, slots = 1, 40
    store, pool, pooled, dense = _setup(device, SMALL, layers, slots)
    lru = pool.attach_device_lru(store)
    _step(SMALL, pooled, dense, 0, 2, 700, device)          # a valid call first
    lru.lru_order[5] = slots + 3
    before = [t.clone() for t in (pool.slot_table, lru.slot_owner, lru.lru_order, lru.counters)]
    layer = pooled[0]
    x = assemble.tokens_tensor(SMALL, SEED, device, 3, stream=701)
    out = torch.empty_like(x)
    inds = torch.empty((3, layer.top_k), dtype=torch.int32, device=device)
    scores = torch.empty((3, layer.top_k), dtype=x.dtype, device=device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    a = layer.layer_args(x, out, inds, scores)
    a.status = status.data_ptr()
    _lib.check(_lib.lib().vm_moe_layer_lru(a, lru.view(0), stream_handle()))
    torch.cuda.synchronize()
    assert int(status.item()) & 16
    for b, t in zip(before, (pool.slot_table, lru.slot_owner, lru.lru_order, lru.counters)):
        assert torch.equal(b, t)


def test_adaptive_threshold_hands_the_state_back(device):
    """Below threshold 1.0 the plan runs on the host (adaptive_topk.py:76-235):
    a layer with a device LRU hands the state back for the call, gives the
    dense layer's bits (both planned), and its slot table follows the planned
    routes cut to the widest row."""
    from veymoe import adaptive

    layers, slots = 1, 48
    store, pool, pooled, dense = _setup(device, SMALL, layers, slots)
    ref = pool_oracle.LruSlots(slots)
    pool.attach_device_lru(store)
    adaptive.set_threshold(0.6)
    try:
        for step, tokens in enumerate([1, 3, 1, 2]):
            routed = _step(SMALL, pooled, dense, 0, tokens, 500 + step, device)
            width = max(adaptive.last_keeps()[0])
            planned = np.asarray(routed).reshape(tokens, SMALL.top_k)[:, :width].reshape(-1).tolist()
            ref.assign(0, planned)
            assert pool.device_lru is not None
    finally:
        adaptive.set_threshold(1.0)
    table = pool.device_lru.state()[0]
    np.testing.assert_array_equal(table, _expected_table(ref, layers, SMALL.experts))
