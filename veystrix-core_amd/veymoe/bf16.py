"""bfloat16 bit-pattern helpers for NumPy (BF16 travels as uint16, as in the
reference's safetensors reader, models/flashnext/store.py:26-41)."""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(values) -> np.ndarray:
    """Round float32 to bf16 (nearest, ties to even); NaN stays NaN."""
    values = np.asarray(values, dtype=np.float32)
    u = values.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(values)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


def bf16_bits_to_f32(bits) -> np.ndarray:
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)
