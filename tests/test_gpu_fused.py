"""The decode pipelines of one token against each other: the multi-token
kernels (0, the default), the one-token front with the gate/up grid and the
down kernel (1), and the front with the experts grid's tagged hand-off (2).  The
same arithmetic, so the same bits, for dense and pooled layers, with and
without a shared expert, layer 0 (generic combine) and later layers (fused
combine), the stream injection, unresolved experts and the device-LRU route
mode; and against the oracle at the layer tolerance.  Pipelines 1 and 2 are
compiled only into a library built with -DVM_FUSED_PIPELINES=1; without them
these tests run the default pipeline alone (the oracle checks, repeats, the
injection formula, the status bit and the device-LRU state), so its shapes
here (hidden 256 with a shared expert, intermediate 384, the reference
checkpoint's 2560/640) stay covered."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import assert_close, host, pooled_stack
from oracle import moe_oracle as mo
from veymoe import _lib, assemble, synth
from veymoe.device import stream_handle
from veymoe.pool import ExpertPool

pytestmark = pytest.mark.gpu

SHAPES = [
    synth.CONFIGS["decode_small"],                                  # 1024/256, 64 experts top-4, no shared
    synth.LayerSpec("fused_s", 256, 128, 64, 4, 128, 1),            # small hidden, shared expert
    synth.LayerSpec("fused_m", 512, 384, 96, 7, 384, 1),            # intermediate not a power of two
    synth.LayerSpec("fused_w", 2560, 640, 128, 10, 640, 1),         # the reference checkpoint's widths
]


def _pipeline(mode):
    return _lib.lib().vm_decode_pipeline(mode)


# the default pipeline first, then the others where the library carries them
MODES = (0, 1, 2) if _lib.lib_built_with_fused_pipelines() else (0,)


def _both(layer, x):
    """(output, inds, scores) of every pipeline, the default first."""
    res = []
    for mode in MODES:
        prev = _pipeline(mode)
        try:
            y = layer(x[None])[0]
            torch.cuda.synchronize()
            res.append((y.clone(), layer.last_inds.clone(), layer.last_scores.clone()))
        finally:
            _pipeline(prev)
    return res


def _same(a, b, what):
    assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b), what


@pytest.mark.parametrize("spec", SHAPES, ids=lambda s: s.name)
@pytest.mark.parametrize("layer_id", [0, 3])
def test_fused_equals_three_launch_dense(device, spec, layer_id):
    seed = 900 + layer_id
    layer = assemble.build_layer(spec, seed, device, layer=layer_id, dense=True)
    for stream in range(3):
        x = assemble.tokens_tensor(spec, seed, device, 1, stream=stream)
        (yf, inf, scf), *others = _both(layer, x)
        for y3, in3, sc3 in others:
            _same(inf, in3, "inds")
            _same(scf, sc3, "scores")
            _same(yf, y3, (spec.name, layer_id, stream))
    ref = mo.moe_layer(mo.bf16_bits_to_f32(synth.tokens(spec, seed, 1, stream=2)),
                       synth.numpy_layer(spec, seed, layer_id), "bf16")
    np.testing.assert_array_equal(host(inf).astype(np.int64), ref["inds"])
    assert_close(host(yf), ref["output"], f"{spec.name} fused decode")


def test_fused_full_layer_through_the_pool(device):
    """hidden 2048 / inter 512 / 512 experts top-10 + shared, every expert at a
    random slot of a pool behind the slot table (the benchmark's layer)."""
    spec = synth.CONFIGS["decode"]
    seed = 2027
    pool = ExpertPool(spec.layout, 2 * spec.experts + 40, layers=2, experts=spec.experts, device=device)
    layers = [assemble.build_layer(spec, seed, device, layer=l, pool=pool) for l in (0, 1)]
    for l, layer in enumerate(layers):
        for stream in range(4):
            x = assemble.tokens_tensor(spec, seed, device, 1, stream=10 * l + stream)
            (yf, inf, scf), *others = _both(layer, x)
            for y3, in3, sc3 in others:
                _same(inf, in3, "inds")
                _same(scf, sc3, "scores")
                _same(yf, y3, (l, stream))
        ref = mo.moe_layer(mo.bf16_bits_to_f32(synth.tokens(spec, seed, 1, stream=10 * l + 3)),
                           synth.numpy_layer(spec, seed, l), "bf16")
        np.testing.assert_array_equal(host(inf).astype(np.int64), ref["inds"])
        assert_close(host(yf), ref["output"], f"layer {l} fused decode through the pool")


def test_fused_injection_and_repeat(device):
    """The stream injection in the combine, and two calls in a row (the
    hand-off words are zeroed by every call's front kernel)."""
    spec = SHAPES[1]
    seed = 77
    layer = assemble.build_layer(spec, seed, device, layer=2, dense=True)
    x = assemble.tokens_tensor(spec, seed, device, 1, stream=4)
    hc = 3
    gen = torch.Generator(device=device).manual_seed(5)
    streams = torch.randn((1, hc * spec.hidden), device=device, generator=gen).to(torch.bfloat16)
    weights = torch.rand((1, hc), device=device, generator=gen).to(torch.bfloat16)
    outs = []
    for mode in (0, 0) + tuple(m for m in MODES[1:] for _ in range(2)):
        prev = _pipeline(mode)
        try:
            target = torch.empty_like(streams)
            y = layer.forward(x, inject=(streams, weights, target))
            torch.cuda.synchronize()
            outs.append((y.clone(), target.clone()))
        finally:
            _pipeline(prev)
    for y, t in outs[1:]:
        _same(y, outs[0][0], "output")
        _same(t, outs[0][1], "injected streams")
    want = (streams.float().view(hc, -1) + (outs[0][0].float() * weights.float().view(hc, 1)).to(torch.bfloat16)
            .float()).to(torch.bfloat16)
    _same(outs[0][1].view(hc, -1), want, "injection formula")


def test_fused_unresolved_expert_sets_status_and_matches(device):
    """A slot-table entry of -1: status bit 0, the slot contributes zeros, the
    same output bits as the three-launch path."""
    spec = SHAPES[1]
    seed = 31
    pool = ExpertPool(spec.layout, spec.experts + 4, layers=1, experts=spec.experts, device=device)
    layer = assemble.build_layer(spec, seed, device, pool=pool)
    x = assemble.tokens_tensor(spec, seed, device, 1, stream=0)
    (_, inds, _), *_ = _both(layer, x)
    hole = int(inds[0, 1])
    pool.slot_table[0, hole] = -1
    out = torch.empty_like(x)
    results = []
    for mode in MODES:
        prev = _pipeline(mode)
        try:
            status = torch.zeros(1, dtype=torch.int32, device=device)
            a = layer.layer_args(x, out, torch.empty((1, spec.top_k), dtype=torch.int32, device=device),
                                 torch.empty((1, spec.top_k), dtype=torch.bfloat16, device=device))
            a.status = status.data_ptr()
            _lib.check(_lib.lib().vm_moe_layer(ctypes.byref(a), stream_handle()))
            torch.cuda.synchronize()
            results.append((out.clone(), int(status.item())))
        finally:
            _pipeline(prev)
    for out_m, status_m in results:
        assert status_m & 1 and status_m & 32 == 0
        _same(results[0][0], out_m, "output with an unresolved expert")
    assert torch.isfinite(results[0][0].float()).all()


def test_fused_device_lru_route_mode(device):
    """The device-LRU call feeds the experts grid the routes of its assign
    kernel: same bits and the same LRU state as the three-launch pipeline."""
    spec = synth.LayerSpec("fused_lru", 256, 128, 64, 4, 128, 1)
    runs = []
    for mode in MODES:
        prev = _pipeline(mode)
        try:
            store, pool, pooled, dense = pooled_stack(device, spec, 2, 24, 61)
            lru = pool.attach_device_lru(store)
            outs = []
            for step in range(12):
                layer = step % 2
                x = assemble.tokens_tensor(spec, 61, device, 1, stream=step)
                outs.append(pooled[layer](x[None])[0].clone())
                if step % 4 == 0:
                    want = dense[layer](x[None])[0]
                    _same(outs[-1], want, ("dense", step))
            torch.cuda.synchronize()
            runs.append((outs, [t.copy() for t in lru.state()], lru.stats()))
        finally:
            _pipeline(prev)
    for other in runs[1:]:
        for a, b in zip(runs[0][0], other[0]):
            _same(a, b, "device-LRU output")
        for a, b in zip(runs[0][1], other[1]):
            np.testing.assert_array_equal(a, b)
        assert runs[0][2] == other[2]
    assert runs[0][2]["misses"] > 24
