"""Seeded synthetic layers for the five benchmark configurations.

Distributions (one per part, all seeded per (seed, layer, expert, projection)):
  * packed weights: uint32 words with eight uniform nibbles 0..15;
  * scales: U(0.005, 0.02) rounded to bf16;  biases: U(-0.1, 0.1) rounded to bf16;
  * router weight: N(0, 0.02) bf16;  activations: N(0, 1) bf16;
  * optional router bias log(Zipf(s) pmf) over a seeded permutation of the
    experts, which skews expert popularity (batched-decode configuration).

Per-expert seeding lets a caller materialise only the experts it needs.
Two implementations share the distributions: NumPy (exact, for parity tests)
and torch on the device (for the multi-gigabyte benchmark pools).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

from .bf16 import f32_to_bf16_bits
from .layout import PARTS, RecordLayout, pack_record

_PROJ_ID = {"gate_proj": 0, "up_proj": 1, "down_proj": 2}


@dataclass(frozen=True)
class LayerSpec:
    """One SwiGLU MoE layer shape."""
    name: str
    hidden: int
    inter: int
    experts: int
    top_k: int
    shared_inter: int = 0
    tokens: int = 1
    zipf_s: Optional[float] = None
    layers: int = 1
    group_size: int = 32

    @property
    def layout(self) -> RecordLayout:
        return RecordLayout(self.hidden, self.inter, self.group_size)


CONFIGS: Dict[str, LayerSpec] = {
    # the reference's CPU-runnable case
    "decode_small": LayerSpec("decode_small", 1024, 256, 64, 4, 0, 1),
    # full-size decode layer, all experts resident behind a slot table
    "decode": LayerSpec("decode", 2048, 512, 512, 10, 512, 1),
    # batched decode with Zipf(1.1) expert popularity
    "batched": LayerSpec("batched", 2048, 512, 512, 10, 512, 32, zipf_s=1.1),
    # 2048-token chunked prefill
    "prefill": LayerSpec("prefill", 2048, 512, 512, 10, 512, 2048),
    # 48-layer stack decode through an LRU pool
    "stack": LayerSpec("stack", 2048, 512, 512, 10, 512, 1, zipf_s=1.1, layers=48),
}


def _rng(seed: int, *path: int) -> np.random.Generator:
    return np.random.default_rng([int(seed) & 0xFFFFFFFF, *[int(p) for p in path]])


def q4_projection(rng: np.random.Generator, out_width: int, in_width: int, group_size: int = 32, count=None):
    """(weight uint32 [.., out, in/8], scales bf16 bits, biases bf16 bits)."""
    lead = () if count is None else (count,)
    weight = rng.integers(0, 2 ** 32, size=(*lead, out_width, in_width // 8), dtype=np.uint32)
    meta = (*lead, out_width, in_width // group_size)
    scales = f32_to_bf16_bits(rng.uniform(0.005, 0.02, size=meta).astype(np.float32))
    biases = f32_to_bf16_bits(rng.uniform(-0.1, 0.1, size=meta).astype(np.float32))
    return weight, scales, biases


def expert_parts(spec: LayerSpec, seed: int, layer: int, expert: int):
    """{(proj, part): array} of one routed expert."""
    parts = {}
    layout = spec.layout
    for proj in ("gate_proj", "up_proj", "down_proj"):
        in_width, out_width = layout.in_out(proj)
        w, s, b = q4_projection(_rng(seed, 1, layer, expert, _PROJ_ID[proj]), out_width, in_width,
                                spec.group_size)
        parts[(proj, "weight")], parts[(proj, "scales")], parts[(proj, "biases")] = w, s, b
    return parts


def expert_record(spec: LayerSpec, seed: int, layer: int, expert: int, out=None) -> np.ndarray:
    return pack_record(expert_parts(spec, seed, layer, expert), spec.layout, out)


class LazyExperts:
    """Indexable [expert] -> part array, generated on demand (and cached)."""

    def __init__(self, spec: LayerSpec, seed: int, layer: int, proj: str, part: str):
        self.spec, self.seed, self.layer, self.key = spec, seed, layer, (proj, part)
        self._cache = {}

    def __getitem__(self, expert):
        expert = int(expert)
        if not 0 <= expert < self.spec.experts:
            raise IndexError(f"expert {expert} outside 0..{self.spec.experts - 1}")
        if expert not in self._cache:
            self._cache[expert] = expert_parts(self.spec, self.seed, self.layer, expert)[self.key]
        return self._cache[expert]

    def __len__(self):
        return self.spec.experts


def router_weight(spec: LayerSpec, seed: int, layer: int) -> np.ndarray:
    rng = _rng(seed, 2, layer)
    return f32_to_bf16_bits(rng.normal(0.0, 0.02, size=(spec.experts, spec.hidden)).astype(np.float32))


def router_bias(spec: LayerSpec, seed: int, layer: int) -> Optional[np.ndarray]:
    """log Zipf(s) pmf over a seeded permutation of the experts (fp32), or None."""
    if spec.zipf_s is None:
        return None
    rng = _rng(seed, 3, layer)
    ranks = np.arange(1, spec.experts + 1, dtype=np.float64)
    pmf = ranks ** -spec.zipf_s
    pmf /= pmf.sum()
    bias = np.empty(spec.experts, dtype=np.float32)
    bias[rng.permutation(spec.experts)] = np.log(pmf).astype(np.float32)
    return bias


def shared_parts(spec: LayerSpec, seed: int, layer: int):
    """Shared expert projections ([1, ...] arrays) and its H -> 1 gate, or None."""
    if not spec.shared_inter:
        return None
    out = {}
    for proj in ("gate_proj", "up_proj", "down_proj"):
        if proj == "down_proj":
            in_width, out_width = spec.shared_inter, spec.hidden
        else:
            in_width, out_width = spec.hidden, spec.shared_inter
        out[proj] = q4_projection(_rng(seed, 4, layer, _PROJ_ID[proj]), out_width, in_width,
                                  spec.group_size, count=1)
    out["gate"] = q4_projection(_rng(seed, 5, layer), 1, spec.hidden, spec.group_size, count=1)
    return out


def tokens(spec: LayerSpec, seed: int, count: Optional[int] = None, stream: int = 0) -> np.ndarray:
    """Activations [count, hidden] as bf16 bits, N(0, 1)."""
    count = spec.tokens if count is None else count
    rng = _rng(seed, 6, stream)
    return f32_to_bf16_bits(rng.normal(0.0, 1.0, size=(count, spec.hidden)).astype(np.float32))


def slot_permutation(spec: LayerSpec, seed: int, slots: int) -> np.ndarray:
    """Random permutation: expert e of layer l sits in slot perm[l * E + e]."""
    return _rng(seed, 7).permutation(slots)[: spec.layers * spec.experts].astype(np.int32)


def numpy_layer(spec: LayerSpec, seed: int, layer: int = 0, materialise: bool = False):
    """Layer dict in the form the oracle reads: ``gate_proj/up_proj/down_proj`` as
    (weight, scales, biases) indexable by expert, ``router``, ``router_bias``,
    shared parts, ``top_k`` and ``layer_id``.  Experts are generated lazily
    unless ``materialise``."""
    layer_dict = {"top_k": spec.top_k, "layer_id": int(layer), "router": router_weight(spec, seed, layer),
                  "router_bias": router_bias(spec, seed, layer)}
    for proj in ("gate_proj", "up_proj", "down_proj"):
        if materialise:
            arrays = [np.stack([expert_parts(spec, seed, layer, e)[(proj, part)] for e in range(spec.experts)])
                      for part in ("weight", "scales", "biases")]
            layer_dict[proj] = tuple(arrays)
        else:
            layer_dict[proj] = tuple(LazyExperts(spec, seed, layer, proj, part)
                                     for part in ("weight", "scales", "biases"))
    shared = shared_parts(spec, seed, layer)
    if shared is not None:
        layer_dict["shared_gate_proj"] = shared["gate_proj"]
        layer_dict["shared_up_proj"] = shared["up_proj"]
        layer_dict["shared_down_proj"] = shared["down_proj"]
        layer_dict["shared_expert_gate"] = shared["gate"]
    return layer_dict


__all__ = ["CONFIGS", "LayerSpec", "LazyExperts", "PARTS", "expert_parts", "expert_record", "numpy_layer",
           "q4_projection", "router_bias", "router_weight", "shared_parts", "slot_permutation", "tokens"]
