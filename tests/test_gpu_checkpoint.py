"""GPU: layers loaded from a safetensors checkpoint give the same bits as the
layers built from the same synthetic tensors, with routed experts dense,
resident in the pool, or filled on demand through the device LRU from a slab
pack in pinned host memory."""
import numpy as np
import pytest
import torch

from veymoe import assemble, checkpoint as ck, synth
from veymoe.pool import ExpertPool

pytestmark = pytest.mark.gpu

SEED = 41


def _export(tmp_path, spec, layers):
    tensors = {}
    for layer in layers:
        tensors.update(ck.layer_tensors(synth.numpy_layer(spec, SEED, layer, materialise=True), layer))
    ck.write_safetensors(str(tmp_path / "model.safetensors"), tensors)
    return ck.SafetensorsStore(str(tmp_path))


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("spec", [synth.LayerSpec("ck_small", 256, 128, 64, 4, 128, 1),
                                  synth.LayerSpec("ck_full", 2048, 512, 64, 10, 512, 1)])
def test_checkpoint_layers_match_the_synthetic_layers(device, tmp_path, spec):
    layers = (0, 1)
    store = _export(tmp_path, spec, layers)
    reference = [assemble.build_layer(spec, SEED, device, layer=l, dense=True) for l in layers]
    dense = [ck.load_layer(store, l, spec.top_k, device, dense=True) for l in layers]
    resident_pool = ExpertPool(spec.layout, 2 * spec.experts + 8, layers=2, experts=spec.experts, device=device)
    resident = [ck.load_layer(store, l, spec.top_k, device, pool=resident_pool, resident=True) for l in layers]
    pack_path = str(tmp_path / "experts.slab")
    ck.write_slab_pack(store, {l: range(spec.experts) for l in layers}, pack_path, spec.layout)
    host = ck.SlabPackFile(pack_path, spec.layout).to_host_store()
    lru_pool = ExpertPool(spec.layout, 40, layers=2, experts=spec.experts, device=device)
    on_demand = [ck.load_layer(store, l, spec.top_k, device, pool=lru_pool, host_store=host) for l in layers]
    lru_pool.attach_device_lru(host)
    for step in range(6):
        layer = step % 2
        x = assemble.tokens_tensor(spec, SEED, device, 1 + step % 3, stream=step)[None]
        want = reference[layer](x)
        for variant in (dense, resident, on_demand):
            got = variant[layer](x)
            torch.cuda.synchronize()
            assert _same(got, want), (spec.name, step)
    assert lru_pool.device_lru.stats()["misses"] > 0
