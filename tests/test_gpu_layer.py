"""GPU parity of the router and the whole decode layer against the oracle."""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, bf16_device, host, ulp_diff_bf16
from oracle import moe_oracle as mo
from veymoe import assemble, synth
from veymoe.layout import RecordLayout
from veymoe.pool import ExpertPool, HostRecordStore
from veymoe.router import router_topk

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tokens,experts,hidden,top_k", [(1, 512, 2048, 10), (3, 512, 2048, 10), (8, 64, 1024, 4),
                                                         (2, 40, 256, 7)])
def test_router_topk_matches_oracle(device, tokens, experts, hidden, top_k):
    rng = np.random.default_rng(tokens * 7 + experts)
    w_bits = mo.f32_to_bf16_bits(rng.normal(0, 0.02, (experts, hidden)).astype(np.float32))
    x_np = mo.bf16r(rng.normal(size=(tokens, hidden)).astype(np.float32))
    inds, scores, gates = router_topk(bf16_device(x_np, device), assemble.bf16_tensor(w_bits, device), top_k,
                                      return_gates=True)
    o_inds, o_scores, o_gates = mo.route(x_np, w_bits, top_k, "bf16")
    np.testing.assert_array_equal(inds.cpu().numpy(), o_inds)
    assert ulp_diff_bf16(host(gates), o_gates).max() <= 1
    assert ulp_diff_bf16(host(scores), o_scores).max() <= 1


def test_router_exact_ties_prefer_the_lower_index(device):
    rng = np.random.default_rng(0)
    hidden, experts = 512, 64
    w = rng.normal(0, 0.02, (experts, hidden)).astype(np.float32)
    x_np = mo.bf16r(rng.normal(size=(1, hidden)).astype(np.float32))
    best = int(np.argmax(x_np @ w.T))
    for dup in (5, 40, 63):
        w[dup] = w[best]                       # identical rows -> identical logits and gates
    w_bits = mo.f32_to_bf16_bits(w)
    inds, _ = router_topk(bf16_device(x_np, device), assemble.bf16_tensor(w_bits, device), 6)
    o_inds, _, _ = mo.route(x_np, w_bits, 6, "bf16")
    tied = sorted({best, 5, 40, 63})
    assert inds.cpu().numpy()[0, :4].tolist() == tied
    np.testing.assert_array_equal(inds.cpu().numpy(), o_inds)


def test_router_fp32_mode(device):
    rng = np.random.default_rng(2)
    w_bits = mo.f32_to_bf16_bits(rng.normal(0, 0.02, (512, 2048)).astype(np.float32))
    x_np = rng.normal(size=(2, 2048)).astype(np.float32)
    inds, scores = router_topk(torch.tensor(x_np, device=device), assemble.bf16_tensor(w_bits, device), 10)
    o_inds, o_scores, _ = mo.route(x_np, w_bits, 10, "f32")
    np.testing.assert_array_equal(inds.cpu().numpy(), o_inds)
    np.testing.assert_allclose(host(scores), o_scores, rtol=1e-5, atol=1e-7)


def _check_layer(layer, spec, seed, x_np, mode, device):
    x = bf16_device(x_np, device) if mode == "bf16" else torch.tensor(x_np, device=device)
    y = layer(x[None])[0]
    torch.cuda.synchronize()
    ref = mo.moe_layer(x_np, synth.numpy_layer(spec, seed), mode)
    inds = layer.last_inds.cpu().numpy()
    np.testing.assert_array_equal(inds, ref["inds"])
    if mode == "bf16":
        assert_close(host(y), ref["output"], f"{spec.name} decode output")
    else:
        assert_close(host(y), ref["output"], f"{spec.name} fp32 decode output", rtol=1e-3, atol=1e-4,
                     max_rel=1e-3)
    return y


@pytest.mark.parametrize("tokens", [1, 4, 8])
def test_decode_small_layer_dense(device, tokens):
    spec = synth.CONFIGS["decode_small"]
    seed = 101 + tokens
    layer = assemble.build_layer(spec, seed, device, dense=True)
    x_np = mo.bf16_bits_to_f32(synth.tokens(spec, seed, tokens))
    _check_layer(layer, spec, seed, x_np, "bf16", device)


def test_decode_small_layer_fp32(device):
    spec = synth.CONFIGS["decode_small"]
    layer = assemble.build_layer(spec, 7, device, dense=True)
    x_np = np.random.default_rng(3).normal(size=(2, spec.hidden)).astype(np.float32)
    _check_layer(layer, spec, 7, x_np, "f32", device)


@pytest.fixture(scope="module")
def full_layer(device):
    spec = synth.CONFIGS["decode"]
    seed = 2026
    pool = ExpertPool(spec.layout, 600, layers=1, experts=spec.experts, device=device)
    layer = assemble.build_layer(spec, seed, device, pool=pool)
    return spec, seed, layer, pool


@pytest.mark.parametrize("tokens", [1, 2, 8])
def test_full_decode_layer_through_the_pool(device, full_layer, tokens):
    """hidden 2048 / inter 512 / 512 experts top-10 + shared expert, every
    expert resident at a random slot behind the int32 slot table."""
    spec, seed, layer, pool = full_layer
    table = pool._host_table[0]
    assert (table >= 0).all() and len(set(table.tolist())) == spec.experts
    assert not np.array_equal(table, np.sort(table))   # a real permutation
    x_np = mo.bf16_bits_to_f32(synth.tokens(spec, seed, tokens, stream=tokens))
    _check_layer(layer, spec, seed, x_np, "bf16", device)


def test_full_decode_layer_repeatable(device, full_layer):
    spec, seed, layer, _ = full_layer
    x = assemble.tokens_tensor(spec, seed, device, 1, stream=9)
    first = layer(x[None])
    second = layer(x[None])
    assert torch.equal(first.view(torch.int16), second.view(torch.int16))


def test_pool_misses_are_staged_and_match_the_dense_layer(device):
    """A 16-slot pool in front of 64 experts held in pinned host memory: the
    split decode (router, host LRU + hipMemcpyAsync staging, experts) gives
    the same bits as the dense layer."""
    spec = synth.LayerSpec("miss", 256, 128, 64, 4, 128, 1)
    seed = 77
    layout = spec.layout
    store = HostRecordStore(layout, spec.experts)
    for e in range(spec.experts):
        store.put(0, e, synth.expert_record(spec, seed, 0, e))
    pool = ExpertPool(layout, 16, layers=1, experts=spec.experts, device=device)
    pooled = assemble.build_layer(spec, seed, device, pool=pool, host_store=store)
    dense = assemble.build_layer(spec, seed, device, dense=True)
    for step in range(12):
        x = assemble.tokens_tensor(spec, seed, device, 1, stream=step)
        a = pooled(x[None])
        b = dense(x[None])
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), step
    sw = pooled.switch_mlp
    assert sw.misses > 0 and pool.bytes_staged == sw.misses * layout.record_bytes
    assert pool.usable_slots == 16


def test_layer_zero_combines_generically_and_later_layers_fuse(device):
    """The reference's layer 0 is not on the custom path
    (metal_combines_scores is False for layer_id 0, expert_cache.py:1434-1443),
    so its decode output is ``(y * scores[..., None]).sum(-2)`` with
    elementwise bf16 products (adaptive_topk.py:275-278); later layers take
    the fused combine.  Same weights and input in both: each output equals its
    formula applied, in fp32 with bf16 roundings, to the per-slot expert
    outputs of the same kernels, bit for bit."""
    from veymoe.layer import HipSwitchGLU, MoELayer

    spec = synth.CONFIGS["decode_small"]
    seed = 211
    l0 = assemble.build_layer(spec, seed, device, dense=True)
    sw = l0.switch_mlp
    sw1 = HipSwitchGLU(sw.hidden, sw.inter, sw.num_experts, layer_id=1,
                       projections={"gate_proj": sw.gate_proj, "up_proj": sw.up_proj, "down_proj": sw.down_proj})
    l1 = MoELayer(l0.gate, sw1, l0.top_k)
    assert not sw.metal_combines_scores and sw1.metal_combines_scores
    x = assemble.tokens_tensor(spec, seed, device, 3, stream=5)
    y0 = l0(x[None])[0]
    inds0, scores0 = l0.last_inds.clone(), l0.last_scores.clone()
    y1 = l1(x[None])[0]
    assert torch.equal(inds0, l1.last_inds) and torch.equal(scores0, l1.last_scores)
    # per-slot outputs: the custom path is not taken for layer 0 even with scores
    per_slot = sw(x[:, None, :], inds0[:, None, :], scores=scores0[:, None, :])[:, 0]
    assert per_slot.shape == (3, spec.top_k, spec.hidden) and not sw._last_fused_shared
    d = host(per_slot)
    s = host(scores0)
    fused = np.zeros((3, spec.hidden), np.float32)
    generic = np.zeros_like(fused)
    for j in range(spec.top_k):
        fused = (fused + d[:, j] * s[:, j:j + 1]).astype(np.float32)
        generic = (generic + mo.bf16r(d[:, j] * s[:, j:j + 1])).astype(np.float32)
    np.testing.assert_array_equal(host(y1), mo.bf16r(fused))
    np.testing.assert_array_equal(host(y0), mo.bf16r(generic))
    assert not np.array_equal(host(y0), host(y1))
    ref = mo.moe_layer(mo.bf16_bits_to_f32(synth.tokens(spec, seed, 3, stream=5)), synth.numpy_layer(spec, seed),
                       "bf16")
    assert_close(host(y0), ref["output"], "layer 0 decode output, generic combine")
