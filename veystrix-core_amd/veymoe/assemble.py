"""Assemble device-resident layers from NumPy arrays or seeded synthetic specs."""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import synth
from .executor import Q4G32Projection
from .layer import HipSwitchGLU, MoELayer, QuantizedMLP, RouterLinear
from .layout import PARTS, RecordLayout
from .pool import ExpertPool


def bf16_tensor(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


def word_tensor(words: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(words, dtype=np.uint32).view(np.int32)).to(device)


def projection(weight, scales, biases, device) -> Q4G32Projection:
    return Q4G32Projection(word_tensor(weight, device), bf16_tensor(scales, device), bf16_tensor(biases, device))


def fill_pool_from_spec(pool: ExpertPool, spec: synth.LayerSpec, seed: int, layer: int,
                        slots: Optional[np.ndarray] = None, chunk: int = 64) -> np.ndarray:
    """Write every expert of ``layer`` into the pool (slot of expert e = slots[e],
    default: a seeded random permutation of free slots) and map them."""
    layout = spec.layout
    if slots is None:
        free = np.array(sorted(pool._free), dtype=np.int64)
        rng = np.random.default_rng([seed, 8, layer])
        slots = rng.permutation(free)[: spec.experts]
    slots = np.asarray(slots, dtype=np.int64)
    host = np.zeros((chunk, layout.record_stride), dtype=np.uint8)
    pinned = torch.empty((chunk, layout.record_stride), dtype=torch.uint8).pin_memory()
    for start in range(0, spec.experts, chunk):
        count = min(chunk, spec.experts - start)
        for i in range(count):
            synth.expert_record(spec, seed, layer, start + i, out=host[i])
        pinned[:count].copy_(torch.from_numpy(host[:count]))
        for i in range(count):
            pool.record(int(slots[start + i])).copy_(pinned[i], non_blocking=False)
    pool.place_all(layer, slots[:spec.experts])
    pool.sync_tables()
    return slots


def build_layer(spec: synth.LayerSpec, seed: int, device, *, layer: int = 0, pool: ExpertPool = None,
                dense: bool = False, host_store=None) -> MoELayer:
    """A MoELayer with the synthetic weights of ``spec`` (identical to
    ``synth.numpy_layer(spec, seed, layer)``).  Routed experts are dense arrays
    (``dense=True``) or records in ``pool`` (filled and mapped here unless a
    host store is given, in which case experts stay non-resident until routed)."""
    layer_np = synth.numpy_layer(spec, seed, layer, materialise=dense)
    bias = layer_np.get("router_bias")
    gate = RouterLinear(bf16_tensor(layer_np["router"], device),
                        None if bias is None else torch.from_numpy(bias).to(device))
    if dense:
        projections = {name: projection(*layer_np[name], device) for name in ("gate_proj", "up_proj", "down_proj")}
        switch = HipSwitchGLU(spec.hidden, spec.inter, spec.experts, projections=projections, layer_id=layer,
                              group_size=spec.group_size)
    else:
        if pool is None:
            raise ValueError("a pool-backed layer needs an ExpertPool")
        if host_store is None:
            fill_pool_from_spec(pool, spec, seed, layer)
        switch = HipSwitchGLU(spec.hidden, spec.inter, spec.experts, pool=pool, layer_id=layer,
                              host_store=host_store, group_size=spec.group_size)
    shared_expert = shared_gate = None
    if spec.shared_inter:
        shared_expert = QuantizedMLP(projection(*layer_np["shared_gate_proj"], device),
                                     projection(*layer_np["shared_up_proj"], device),
                                     projection(*layer_np["shared_down_proj"], device))
        shared_gate = projection(*layer_np["shared_expert_gate"], device)
    return MoELayer(gate, switch, spec.top_k, shared_expert=shared_expert, shared_expert_gate=shared_gate,
                    layer_id=layer)


def tokens_tensor(spec: synth.LayerSpec, seed: int, device, count=None, stream=0) -> torch.Tensor:
    return bf16_tensor(synth.tokens(spec, seed, count, stream), device)


# ------------------------------------------------------ device generation --

def random_records_(records: torch.Tensor, layout: RecordLayout, generator: torch.Generator) -> None:
    """Fill a [n, stride] uint8 device view with the synthetic distributions
    (uniform nibbles; scales U(0.005, 0.02); biases U(-0.1, 0.1), bf16) using
    a device generator.  For multi-gigabyte benchmark pools."""
    n = records.shape[0]
    for key in PARTS:
        start, size = layout.offset(*key), layout.sizes[key]
        part = records[:, start:start + size]
        if key[1] == "weight":
            part.copy_(torch.randint(0, 256, (n, size), dtype=torch.uint8, device=records.device,
                                     generator=generator))
        else:
            low, high = (0.005, 0.02) if key[1] == "scales" else (-0.1, 0.1)
            vals = torch.empty((n, size // 2), dtype=torch.float32, device=records.device)
            vals.uniform_(low, high, generator=generator)
            part.copy_(vals.to(torch.bfloat16).view(torch.uint8).reshape(n, size))
