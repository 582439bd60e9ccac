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
