"""Batched decode / chunked prefill (rows > 8) on the grouped kernels."""
from __future__ import annotations


def grouped_layer(layer, flat):
    raise NotImplementedError("the grouped (rows > 8) path is not built yet")
