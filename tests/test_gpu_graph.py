"""HIP-graph replay of decode steps (veymoe.graph.StepGraph) over pools with
the LRU state on the device.

Two identical stacks (same seed): one replays its captured step, the other
issues the same calls eagerly.  Every replay must give the eager outputs bit
for bit, and the dense layers' outputs, and leave the same LRU state (slot
table, owners, queue, counters).  The two runs alternate with host reads of
the state between replays, so a replay that only worked the first time, or
left work behind, would show."""
import pytest
import torch

from gpu_util import pooled_stack
from veymoe import assemble, synth
from veymoe.graph import StepGraph

pytestmark = pytest.mark.gpu

SEED = 91
SMALL = synth.LayerSpec("graph_small", 256, 128, 64, 4, 128, 1)


def _inputs(spec, layers, rows, step, device):
    return torch.stack([assemble.tokens_tensor(spec, SEED, device, rows, stream=1000 * step + l)
                        for l in range(layers)])


@pytest.mark.parametrize("rows", [1, 3])
def test_step_graph_replays_equal_eager_steps_and_the_dense_layers(device, rows):
    layers, slots = 3, 40
    store_a, pool_a, pooled_a, dense = pooled_stack(device, SMALL, layers, slots, SEED)
    store_b, pool_b, pooled_b, _ = pooled_stack(device, SMALL, layers, slots, SEED)
    lru_a = pool_a.attach_device_lru(store_a)
    lru_b = pool_b.attach_device_lru(store_b)
    graph = StepGraph(pooled_a, rows=rows, device=device).capture()
    eager = StepGraph(pooled_b, rows=rows, device=device)
    for step in range(8):
        x = _inputs(SMALL, layers, rows, step, device)
        got = graph.replay(x).clone()
        eager.x.copy_(x)
        want = eager.run_eager().clone()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
        for l in range(layers):
            ref = dense[l](x[l][None])[0]
            assert torch.equal(got[l].view(torch.int16), ref.view(torch.int16)), (step, l)
        for a, b in zip(lru_a.state(), lru_b.state()):
            assert (a == b).all(), step
        assert torch.equal(lru_a.counters, lru_b.counters)
    assert lru_a.stats()["misses"] > slots        # evictions happened inside the replays


def test_step_graph_refuses_host_lru_layers_and_detached_state(device):
    layers, slots = 2, 40
    store, pool, pooled, _ = pooled_stack(device, SMALL, layers, slots, SEED)
    with pytest.raises(ValueError):
        StepGraph(pooled, device=device)            # partly resident, host LRU
    pool.attach_device_lru(store)
    graph = StepGraph(pooled, device=device).capture()
    graph.replay(_inputs(SMALL, layers, 1, 0, device))
    torch.cuda.synchronize()
    pool.detach_device_lru()
    with pytest.raises(RuntimeError):
        graph.replay()


def test_step_graph_survives_a_grouped_call_and_refuses_adaptive_routing(device):
    """A call above the decode bound hands the LRU state to the host and
    uploads it back into the same device buffers, so a graph recorded before
    it replays on: equal to an eager twin that ran the same calls, and to the
    dense layers.  With a threshold below 1.0 (or a route observer) a graph
    would route exactly where the eager call adapts: replay and build raise."""
    from veymoe import adaptive

    layers, slots = 2, 40
    store_a, pool_a, pooled_a, dense = pooled_stack(device, SMALL, layers, slots, SEED)
    store_b, pool_b, pooled_b, _ = pooled_stack(device, SMALL, layers, slots, SEED)
    lru_a = pool_a.attach_device_lru(store_a)
    lru_b = pool_b.attach_device_lru(store_b)
    graph = StepGraph(pooled_a, device=device).capture()
    eager = StepGraph(pooled_b, device=device)
    for step in range(4):
        if step == 2:   # a 12-row call on layer 0 of both stacks
            xg = assemble.tokens_tensor(SMALL, SEED, device, 12, stream=77)
            ga, gb = pooled_a[0](xg[None]), pooled_b[0](xg[None])
            assert torch.equal(ga.view(torch.int16), gb.view(torch.int16))
            assert pool_a.device_lru is lru_a and pool_b.device_lru is lru_b
        x = _inputs(SMALL, layers, 1, step, device)
        got = graph.replay(x).clone()
        eager.x.copy_(x)
        want = eager.run_eager().clone()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
        for l in range(layers):
            ref = dense[l](x[l][None])[0]
            assert torch.equal(got[l].view(torch.int16), ref.view(torch.int16)), (step, l)
        for a, b in zip(lru_a.state(), lru_b.state()):
            assert (a == b).all(), step
    try:
        adaptive.set_layer_thresholds({1: 0.5})
        with pytest.raises(RuntimeError):
            graph.replay()
        with pytest.raises(RuntimeError):
            StepGraph(pooled_a, device=device)
        adaptive.set_layer_thresholds()
        adaptive.set_route_observer(lambda *a: None)
        with pytest.raises(RuntimeError):
            graph.replay()
    finally:
        adaptive.set_layer_thresholds()
        adaptive.set_route_observer()
    graph.replay()
    torch.cuda.synchronize()
