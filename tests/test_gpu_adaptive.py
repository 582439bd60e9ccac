"""GPU: adaptive top-k through MoELayer (router-only call with the gates, host
plan, experts-only call) against the oracle's adaptive routing
(adaptive_topk.py:76-262), and the split path of fp32 calls above the decode
bound, whose chunks each keep their own workspace between the two calls."""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, bf16_device, host
from oracle import moe_oracle as mo
from veymoe import adaptive, assemble, synth
from veymoe.pool import ExpertPool, HostRecordStore

pytestmark = pytest.mark.gpu

SPEC = synth.LayerSpec("adaptive", 1024, 256, 64, 8, 256, 1)


@pytest.fixture(autouse=True)
def _reset():
    yield
    adaptive.set_threshold(1.0)
    adaptive.set_min_keep(1)
    adaptive.set_resident_experts()
    adaptive.set_route_observer()
    adaptive.reset_keep_stats()


def _near_tie(gates_row, k):
    order = np.sort(mo.f32_to_bf16_bits(np.asarray(gates_row, np.float32)).astype(np.int64))[::-1]
    return order[k - 1] - order[k] <= 1


@pytest.mark.parametrize("tokens,blend", [(1, 1.0), (6, 1.0), (40, 1.0), (130, 1.0), (6, 0.3), (130, 0.3)],
                         ids=["decode-1", "decode-6", "rows-40", "grouped-130", "decode-6-blend0.3",
                              "grouped-130-blend0.3"])
def test_adaptive_layer_against_the_oracle(device, tokens, blend):
    """Blend 0.3 (FLASHNEXT_RENORM_BLEND) renormalises over a mix of the kept
    and the top-k mass, with blend rounded to bf16 as the reference does."""
    seed = 410 + tokens
    adaptive.set_threshold(0.6)
    adaptive.set_min_keep(2)
    layer = assemble.build_layer(SPEC, seed, device, dense=True)
    layer.renorm_blend = blend
    x_np = mo.bf16_bits_to_f32(synth.tokens(SPEC, seed, tokens))
    y = host(layer(bf16_device(x_np, device)))
    torch.cuda.synchronize()
    path = "decode" if tokens <= 8 else "prefill"
    ref = mo.moe_layer(x_np, synth.numpy_layer(SPEC, seed), "bf16", path=path,
                       adaptive=dict(threshold=0.6, min_keep=2, blend=blend))
    width = ref["inds"].shape[1]
    inds = layer.last_inds.cpu().numpy()
    same = (inds[:, :width] == ref["inds"]).all(axis=1)
    if not same.all():   # only rows whose top-k differs from the oracle's by a near tie
        _, _, gates = mo.route(x_np[~same], synth.numpy_layer(SPEC, seed)["router"], SPEC.top_k, "bf16")
        for g in gates:
            assert _near_tie(g, SPEC.top_k)
    assert (~same).sum() <= max(1, tokens // 50)
    keeps = adaptive.last_keeps()[0]
    assert len(keeps) == tokens and min(keeps) >= 2 and min(keeps) < SPEC.top_k   # some slots dropped
    np.testing.assert_array_equal(layer.last_scores.float().cpu().numpy()[same, width:], 0.0)
    if tokens <= 8:
        assert_close(y[same], ref["output"][same], f"adaptive decode T={tokens}")
    else:
        assert mo.max_abs_rel(y[same], ref["output"][same]) <= 2.0 ** -7, mo.max_abs_rel(y[same], ref["output"][same])


def test_adaptive_pool_equals_dense_and_counts_the_planned_routes(device):
    """A 16-slot pool in front of 64 experts in pinned host memory, threshold
    0.5: the pooled layer gives the dense layer's bits, and its LRU pass sees
    the planned routes cut to the widest row."""
    seed = 431
    layout = SPEC.layout
    store = HostRecordStore(layout, SPEC.experts)
    for e in range(SPEC.experts):
        store.put(0, e, synth.expert_record(SPEC, seed, 0, e))
    pool = ExpertPool(layout, 16, layers=1, experts=SPEC.experts, device=device)
    pooled = assemble.build_layer(SPEC, seed, device, pool=pool, host_store=store)
    dense = assemble.build_layer(SPEC, seed, device, dense=True)
    adaptive.set_threshold(0.5)
    routed = 0
    for step in range(8):
        x = assemble.tokens_tensor(SPEC, seed, device, 1, stream=step)
        a = pooled(x[None])
        b = dense(x[None])
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), step
        keeps = adaptive.last_keeps()[0]
        routed += max(keeps)   # one row: the width is its keep
    sw = pooled.switch_mlp
    assert sw.hits + sw.misses == routed and sw.misses > 0


def test_fp32_split_path_above_the_decode_bound(device):
    """fp32 rows above the decode bound run the decode kernels in chunks of 8
    rows.  A router-only call followed by an experts-only call (a pool that
    does not hold every expert) must leave every chunk's routes and shared
    gate in place between the two: 12 rows through a pool that starts empty
    (the first call stages its misses between the router and the experts)
    give the dense layer's bits."""
    seed = 433
    layout = SPEC.layout
    store = HostRecordStore(layout, SPEC.experts)
    for e in range(SPEC.experts):
        store.put(0, e, synth.expert_record(SPEC, seed, 0, e))
    pool = ExpertPool(layout, SPEC.experts, layers=1, experts=SPEC.experts, device=device)
    pooled = assemble.build_layer(SPEC, seed, device, pool=pool, host_store=store)
    dense = assemble.build_layer(SPEC, seed, device, dense=True)
    x = torch.from_numpy(np.random.default_rng(5).normal(size=(12, SPEC.hidden)).astype(np.float32)).to(device)
    a = pooled(x)
    b = dense(x)
    assert pooled.switch_mlp.misses > 0
    assert torch.equal(a, b)
    # and under the adaptive plan, in fp32 steps
    adaptive.set_threshold(0.6)
    c = pooled(x)
    d = dense(x)
    assert torch.equal(c, d)
    ref = mo.moe_layer(x.cpu().numpy(), synth.numpy_layer(SPEC, seed), "f32", adaptive=dict(threshold=0.6))
    assert_close(host(d), ref["output"], "adaptive fp32 chunks", rtol=1e-3, atol=1e-4, max_rel=1e-3)


def test_route_observer_at_threshold_one_leaves_the_routes(device):
    """An observer at the default threshold sees each call's routes with keep
    k, and the layer's output is the plain one."""
    seed = 437
    layer = assemble.build_layer(SPEC, seed, device, dense=True)
    x = assemble.tokens_tensor(SPEC, seed, device, 3)
    plain = layer(x)
    plain_inds = layer.last_inds.clone()
    seen = []
    adaptive.set_route_observer(lambda l, e, w, k: seen.append((l, e, w, k)))
    observed = layer(x)
    assert torch.equal(plain.view(torch.int16), observed.view(torch.int16))
    assert len(seen) == 1 and seen[0][0] == 0 and seen[0][3] == [SPEC.top_k] * 3
    assert seen[0][1] == plain_inds.cpu().tolist()
