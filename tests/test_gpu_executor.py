"""GPU parity of the executor (vm_moe_execute) against the oracle.

Cases follow the reference's MLX smoke tests (models/flashnext/tests/unit/
test_metal_runtime.py:358-836), with the oracle standing in for gather_qmm.
"""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, bf16_device, host, packs, to_device
from oracle import moe_oracle as mo
from veymoe import HipMoEExecutor, weighted_combine
from veymoe.assemble import word_tensor
from veymoe.layout import HEADER, RecordLayout, pack_record

pytestmark = pytest.mark.gpu


def _oracle_packs(np_packs):
    return {name: tuple(parts) for name, parts in np_packs.items()}


def _pattern(n, mod, center, scale):
    return ((np.arange(n, dtype=np.float32) % mod) - center) / scale


def test_weighted_combine_known_answer(device):
    outputs = torch.tensor([[[1.0, 2.0], [10.0, 20.0], [100.0, 200.0]],
                            [[3.0, 4.0], [30.0, 40.0], [300.0, 400.0]]], device=device)
    routes = torch.tensor([[2, 0], [1, 2]], dtype=torch.int32, device=device)
    scores = torch.tensor([[0.25, 0.75], [0.4, 0.6]], device=device)
    expected = np.array([[25.75, 51.5], [192.0, 256.0]], np.float32)
    np.testing.assert_array_equal(host(weighted_combine(outputs, routes, scores)), expected)
    ex = HipMoEExecutor(3, 2, 2)
    np.testing.assert_array_equal(host(ex.execute(outputs, routes, scores)), expected)
    assert ex.last_path == "hip"


def test_tiny_q4g32_path_stays_within_tolerance(device):
    np_packs = packs(0, 32, 32, 2)
    x_np = mo.bf16r(_pattern(32, 13, 6, 8)).reshape(1, 32)
    routes = np.array([[0, 1]], np.int32)
    scores = np.array([[0.25, 0.75]], np.float32)
    ex = HipMoEExecutor(2, 32, 2)
    dev = to_device(np_packs, device)
    x = bf16_device(x_np, device)
    r = torch.tensor(routes, device=device)
    s = torch.tensor(scores, device=device)
    per_slot = ex.execute(x, r, dev)
    fused = ex.execute(x, r, dev, scores=s)
    _, _, _, down, expected = mo.execute(x_np, routes, _oracle_packs(np_packs), "bf16", scores=scores)
    assert ex.last_path == "hip"
    assert_close(host(per_slot), down, "per-slot down diverged")
    assert_close(host(weighted_combine(per_slot, r, s)), mo.weighted_combine(down, routes, scores), "weighted")
    assert_close(host(fused), expected, "fused down and route output diverged")


def test_wide_shapes_two_tokens_three_routes(device):
    np_packs = packs(1, 256, 128, 4)
    x_np = mo.bf16r(_pattern(512, 29, 14, 16)).reshape(2, 256)
    routes = np.array([[0, 2, 3], [3, 1, 0]], np.int32)
    scores = np.array([[0.2, 0.3, 0.5], [0.5, 0.25, 0.25]], np.float32)
    ex = HipMoEExecutor(4, 256, 3, max_width=256)
    out = ex.execute(bf16_device(x_np, device), torch.tensor(routes, device=device), to_device(np_packs, device),
                     scores=torch.tensor(scores, device=device))
    *_, expected = mo.execute(x_np, routes, _oracle_packs(np_packs), "bf16", scores=scores)
    assert_close(host(out), expected, "wide Q4/G32 output diverged")


@pytest.mark.parametrize("hidden,inter,experts,top_k", [(2560, 640, 2, 2), (2048, 512, 4, 4), (1024, 256, 8, 4)])
def test_production_shapes_bf16(device, hidden, inter, experts, top_k):
    np_packs = packs(2, hidden, inter, experts)
    x_np = mo.bf16r(_pattern(hidden, 31, 15, 64)).reshape(1, hidden)
    routes = np.arange(top_k, dtype=np.int32).reshape(1, top_k)
    scores = mo.bf16r(np.arange(1, top_k + 1, dtype=np.float32) / (top_k * (top_k + 1) / 2)).reshape(1, top_k)
    ex = HipMoEExecutor(experts, hidden, top_k)
    out = ex.execute(bf16_device(x_np, device), torch.tensor(routes, device=device), to_device(np_packs, device),
                     scores=bf16_device(scores, device))
    *_, expected = mo.execute(x_np, routes, _oracle_packs(np_packs), "bf16", scores=scores)
    assert_close(host(out), expected, f"{hidden}x{inter} bf16 output diverged")


@pytest.mark.parametrize("hidden,inter,experts,top_k", [(256, 128, 4, 3), (2560, 640, 8, 7), (2048, 512, 12, 10)])
def test_float32_activations_match_the_fp32_oracle(device, hidden, inter, experts, top_k):
    """fp32 activations with bf16 metadata: rtol 1e-3 / atol 1e-4 against the
    fp32-accumulation oracle (test_metal_runtime.py:516-639)."""
    np_packs = packs(3, hidden, inter, experts)
    x_np = _pattern(hidden, 31, 15, 64).reshape(1, hidden)
    routes = np.arange(top_k, dtype=np.int32).reshape(1, top_k) % experts
    scores = np.arange(1, top_k + 1, dtype=np.float32)
    scores = (scores / scores.sum()).reshape(1, top_k)
    ex = HipMoEExecutor(experts, hidden, top_k)
    out = ex.execute(torch.tensor(x_np, device=device), torch.tensor(routes, device=device),
                     to_device(np_packs, device), scores=torch.tensor(scores, device=device))
    *_, expected = mo.execute(x_np, routes, _oracle_packs(np_packs), "f32", scores=scores)
    assert_close(host(out), expected, "fp32 output diverged", rtol=1e-3, atol=1e-4, max_rel=1e-3)


def test_adaptive_widths_one_through_ten(device):
    np_packs = packs(4, 32, 32, 16)
    x_np = _pattern(32, 17, 8, 16).reshape(1, 32)
    dev = to_device(np_packs, device)
    for width in range(1, 11):
        routes = np.arange(width, dtype=np.int32).reshape(1, width)
        scores = np.arange(1, width + 1, dtype=np.float32).reshape(1, width)
        scores /= scores.sum()
        out = HipMoEExecutor(16, 32, width).execute(torch.tensor(x_np, device=device),
                                                    torch.tensor(routes, device=device), dev,
                                                    scores=torch.tensor(scores, device=device))
        *_, expected = mo.execute(x_np, routes, _oracle_packs(np_packs), "f32", scores=scores)
        assert_close(host(out), expected, f"width {width}", rtol=1e-3, atol=1e-4, max_rel=1e-3)


def _shared_case(device):
    hidden, inter = 2560, 640
    np_packs = packs(5, hidden, inter, 2)
    x = bf16_device(_pattern(hidden, 31, 15, 64).reshape(1, hidden), device)
    routes = torch.tensor([[0, 1]], dtype=torch.int32, device=device)
    scores = torch.tensor([[0.375, 0.625]], device=device)
    shared = bf16_device(_pattern(hidden, 29, 14, 32).reshape(1, hidden), device)
    return HipMoEExecutor(2, hidden, 2), x, routes, scores, to_device(np_packs, device), shared


def test_fused_shared_y_is_bit_identical(device):
    ex, x, routes, scores, dev, shared_y = _shared_case(device)
    unfused = ex.execute(x, routes, dev, scores=scores)
    fused = ex.execute(x, routes, dev, scores=scores, shared_y=shared_y)
    expected = (unfused.float() + shared_y.float()).to(torch.bfloat16)
    assert torch.equal(fused.view(torch.int16), expected.view(torch.int16))


def test_fused_shared_parts_preserve_bf16_product_rounding(device):
    ex, x, routes, scores, dev, shared = _shared_case(device)
    gate = torch.tensor([[0.333984375]], dtype=torch.bfloat16, device=device)
    unfused = ex.execute(x, routes, dev, scores=scores)
    fused = ex.execute(x, routes, dev, scores=scores, shared=shared, shared_gate=gate)
    product = (shared.float() * gate.float()).to(torch.bfloat16)
    expected = (unfused.float() + product.float()).to(torch.bfloat16)
    assert torch.equal(fused.view(torch.int16), expected.view(torch.int16))


def _records(np_packs, layout, experts):
    rec = np.zeros((experts, layout.record_stride), np.uint8)
    for e in range(experts):
        parts = {(name, part): np_packs[name][i][e] for name in np_packs
                 for i, part in enumerate(("weight", "scales", "biases"))}
        pack_record(parts, layout, rec[e])
    return rec


def test_slab_pack_and_stream_pack_records_are_bit_identical(device):
    hidden, inter, experts = 2048, 512, 3
    np_packs = packs(6, hidden, inter, experts)
    layout = RecordLayout(hidden, inter)
    rec = _records(np_packs, layout, experts)
    slab = torch.zeros(HEADER + experts * layout.record_stride, dtype=torch.uint8)
    # slot s holds expert (s + 1) % experts
    for s in range(experts):
        slab[HEADER + s * layout.record_stride: HEADER + (s + 1) * layout.record_stride] = \
            torch.from_numpy(rec[(s + 1) % experts])
    slab = slab.to(device)
    stream = torch.from_numpy(rec.reshape(-1)).to(device)
    dev = to_device(np_packs, device)
    x = bf16_device(mo.bf16r(_pattern(hidden, 31, 15, 64)).reshape(1, hidden), device)
    scores = torch.tensor([[0.375, 0.625]], device=device)
    ex = HipMoEExecutor(experts, hidden, 2)
    expected = ex.execute(x, torch.tensor([[2, 0]], dtype=torch.int32, device=device), dev, scores=scores)
    slot_words = word_tensor(np.array([[0x80000000 | 1, 0x80000000 | 2]], np.uint32), device)
    from_slab = ex.execute(x, slot_words, dev, scores=scores, slab_pack=slab)
    assert torch.equal(from_slab.view(torch.int16), expected.view(torch.int16))
    mixed = word_tensor(np.array([[2, 0x80000000 | 2]], np.uint32), device)
    from_stream = ex.execute(x, mixed, dev, scores=scores, slab_pack=slab, stream_pack=stream)
    assert torch.equal(from_stream.view(torch.int16), expected.view(torch.int16))
    # precomputed activations (the reference's decode overlap) give the same bits
    act = ex.pool_activations(x, slot_words, (dev["gate_proj"], dev["up_proj"], dev["down_proj"]), slab)
    overlapped = ex.execute(x, slot_words, dev, scores=scores, slab_pack=slab, pool_activation=act)
    assert torch.equal(overlapped.view(torch.int16), expected.view(torch.int16))


def test_return_all_matches_oracle_projections(device):
    np_packs = packs(7, 1024, 256, 4)
    x_np = mo.bf16r(np.random.default_rng(1).normal(size=(2, 1024)).astype(np.float32))
    routes = np.array([[1, 3], [0, 1]], np.int32)
    ex = HipMoEExecutor(4, 1024, 2)
    g, u, d = ex.execute(bf16_device(x_np, device), torch.tensor(routes, device=device), to_device(np_packs, device),
                         return_all=True)
    og, ou, _, od, _ = mo.execute(x_np, routes, _oracle_packs(np_packs), "bf16")
    assert_close(host(g), og, "gate")
    assert_close(host(u), ou, "up")
    assert_close(host(d), od, "down")


def test_out_of_range_routes_set_the_status_flag(device):
    np_packs = packs(8, 256, 128, 4)
    ex = HipMoEExecutor(4, 256, 2)
    x = bf16_device(np.ones((1, 256), np.float32), device)
    out = ex.execute(x, torch.tensor([[1, 9]], dtype=torch.int32, device=device), to_device(np_packs, device),
                     scores=torch.tensor([[0.5, 0.5]], device=device))
    torch.cuda.synchronize()
    assert ex.status() & 1
    assert torch.isfinite(out.float()).all()
    ex.execute(x, torch.tensor([[1, 2]], dtype=torch.int32, device=device), to_device(np_packs, device))
    assert ex.status() == 0
