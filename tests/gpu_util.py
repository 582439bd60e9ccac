"""Helpers shared by the GPU parity tests (not collected by pytest)."""
import numpy as np
import torch

from oracle import moe_oracle as mo
from veymoe import assemble, synth


def packs(seed, hidden, inter, experts):
    """Random Q4/G32 projections (numpy) in the synthetic distributions."""
    rng = np.random.default_rng(seed)
    return {
        "gate_proj": synth.q4_projection(rng, inter, hidden, count=experts),
        "up_proj": synth.q4_projection(rng, inter, hidden, count=experts),
        "down_proj": synth.q4_projection(rng, hidden, inter, count=experts),
    }


def to_device(np_packs, device):
    return {name: assemble.projection(*parts, device) for name, parts in np_packs.items()}


def bf16_device(values, device):
    return torch.tensor(np.asarray(values, np.float32), device=device).to(torch.bfloat16)


def host(t):
    return t.float().cpu().numpy()


def assert_close(actual, expected, message, rtol=2e-2, atol=3e-3, min_cosine=0.9999, max_rel=2e-2):
    """The reference's tolerance (test_metal_runtime.py:321-350) plus the
    max-abs-rel bound: max|a - e| / max|e| <= max_rel."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    np.testing.assert_allclose(actual, expected, rtol=rtol, atol=atol, err_msg=message)
    if max_rel is not None:
        assert mo.max_abs_rel(actual, expected) <= max_rel, (message, mo.max_abs_rel(actual, expected))
    na, ne = np.linalg.norm(actual), np.linalg.norm(expected)
    if na > 0 and ne > 0:
        cosine = float((actual * expected).sum() / (na * ne))
        assert cosine >= min_cosine, (message, cosine)


def ulp_diff_bf16(a, b):
    """|bit distance| between bf16 values given as float arrays."""
    ia = mo.f32_to_bf16_bits(np.asarray(a, np.float32)).astype(np.int32)
    ib = mo.f32_to_bf16_bits(np.asarray(b, np.float32)).astype(np.int32)
    return np.abs(ia - ib)


def pooled_stack(device, spec, layers, slots, seed):
    """A pinned host store with every (layer, expert) record of ``spec``, an
    empty pool of ``slots`` records, pool-backed layers over it and the same
    layers with dense weights: (store, pool, pooled, dense)."""
    from veymoe.pool import ExpertPool, HostRecordStore

    store = HostRecordStore(spec.layout, layers * spec.experts)
    for layer in range(layers):
        for expert in range(spec.experts):
            store.put(layer, expert, synth.expert_record(spec, seed, layer, expert))
    pool = ExpertPool(spec.layout, slots, layers=layers, experts=spec.experts, device=device)
    pooled = [assemble.build_layer(spec, seed, device, layer=l, pool=pool, host_store=store) for l in range(layers)]
    dense = [assemble.build_layer(spec, seed, device, layer=l, dense=True) for l in range(layers)]
    return store, pool, pooled, dense
