"""GPU: a layer-major window through real MoE layers gives the chunk-major
bits (every chunk of the window in one grouped call per layer; a tiny tail
chunk on the decode path afterwards)."""
import pytest
import torch

from veymoe import assemble, layer_major as lm, synth
from veymoe.pool import ExpertPool

pytestmark = pytest.mark.gpu

SPEC = synth.LayerSpec("window", 256, 128, 64, 4, 128, 1)
SEED = 5


def _residual(i, x, y):
    return (x.float() + y.float()).to(torch.bfloat16)


def test_window_equals_chunk_major(device):
    pool = ExpertPool(SPEC.layout, 3 * SPEC.experts, layers=3, experts=SPEC.experts, device=device)
    layers = [assemble.build_layer(SPEC, SEED, device, layer=l, pool=pool) for l in range(3)]
    chunks = [assemble.tokens_tensor(SPEC, SEED, device, n, stream=k) for k, n in enumerate((80, 96, 72, 130, 5))]
    ref = lm.run_chunk_major(layers, chunks, _residual)
    got = lm.run_window(layers, chunks, _residual)
    torch.cuda.synchronize()
    assert len(got) == len(ref)
    for k, (a, b) in enumerate(zip(got, ref)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), k


def _full_layers(count, device, seed):
    """Full-width layers (hidden 2048, inter 512, 512 experts top-10 + shared)
    over one pool of device-generated records at a seeded permutation of slots."""
    import numpy as np

    from veymoe.layer import HipSwitchGLU, MoELayer, QuantizedMLP, RouterLinear

    spec = synth.CONFIGS["prefill"]
    pool = ExpertPool(spec.layout, count * spec.experts, layers=count, experts=spec.experts, device=device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    view = pool.buffer[pool.header_size:].view(pool.slots, spec.layout.record_stride)
    for start in range(0, pool.slots, 256):
        assemble.random_records_(view[start:start + 256], spec.layout, gen)
    perm = np.random.default_rng(seed).permutation(pool.slots)
    layers = []
    for l in range(count):
        pool.place_all(l, perm[l * spec.experts:(l + 1) * spec.experts])
        np_layer = synth.numpy_layer(spec, seed, l)
        shared = QuantizedMLP(*(assemble.projection(*np_layer[n], device)
                                for n in ("shared_gate_proj", "shared_up_proj", "shared_down_proj")))
        switch = HipSwitchGLU(spec.hidden, spec.inter, spec.experts, pool=pool, layer_id=l)
        layers.append(MoELayer(RouterLinear(assemble.bf16_tensor(np_layer["router"], device)), switch, spec.top_k,
                               shared_expert=shared,
                               shared_expert_gate=assemble.projection(*np_layer["shared_expert_gate"], device)))
    pool.sync_tables()
    return spec, layers


def test_full_shape_window_of_four_2048_row_chunks_equals_chunk_major(device):
    """The layer-major window at the prefill shape: four 2048-row chunks
    (8,192 rows per grouped call) through three full-width layers give the
    chunk-major bits."""
    spec, layers = _full_layers(3, device, 808)
    chunks = [assemble.tokens_tensor(spec, 808, device, 2048, stream=k) for k in range(4)]
    ref = lm.run_chunk_major(layers, chunks, _residual)
    got = lm.run_window(layers, chunks, _residual)
    torch.cuda.synchronize()
    assert len(got) == len(ref) == 4
    for k, (a, b) in enumerate(zip(got, ref)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), k
