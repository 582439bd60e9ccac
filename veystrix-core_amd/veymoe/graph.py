"""One decode step through a stack of MoE layers, recorded once as a HIP graph.

The reference drives its decode loop layer by layer from the host, and must:
every layer syncs its routes to the host for the LRU pass before the experts
run (expert_cache.py:1738-1749, 1842-1947).  Here a layer whose pool keeps its
LRU state on the device (``ExpertPool.attach_device_lru``), or whose experts
are all resident, issues only kernels on one stream: router, selection and
assign, miss fill, experts.  A whole step over every layer is then one graph,
so the host launches one graph per token instead of ~5 kernels per layer.

``StepGraph`` owns static buffers: ``x`` [layers, rows, hidden] (the input of
every layer for the step), ``out``, ``inds`` and ``scores``.  ``replay(x)``
copies the step's inputs in and launches the graph; the device LRU state moves
on exactly as with eager calls.  Layers whose pool would need the host LRU
(partly resident, no device LRU) are refused, and so is a replay after a
pool's device LRU was detached and not attached again over the same buffers.
A graph records exact top-k routing, so building or replaying one while
adaptive routing (a threshold below 1.0) or a route observer is active for
any of its layers raises: the eager layer call would route differently.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _lib, adaptive
from .device import stream_handle
from .layer import MAX_DECODE_ROWS, MoELayer


def _refuse_adaptive(layers) -> None:
    if adaptive.observing():
        raise RuntimeError("a step graph records exact routing: clear the route observer first")
    for i, layer in enumerate(layers):
        if adaptive.threshold_for(layer._flashnext_layer_id) < 1.0:
            raise RuntimeError(f"a step graph records exact routing: layer {i} has an adaptive threshold below 1.0")


def _device_only(layer: MoELayer) -> bool:
    sw = layer.switch_mlp
    return sw.pool is None or sw.pool.device_lru is not None or sw._pool_fully_resident()


class StepGraph:
    """A decode step (``rows`` tokens) through ``layers`` as one HIP graph."""

    def __init__(self, layers: Sequence[MoELayer], rows: int = 1, dtype=torch.bfloat16, device=None):
        layers = list(layers)
        if not layers:
            raise ValueError("a step needs at least one layer")
        if not 1 <= rows <= MAX_DECODE_ROWS:
            raise ValueError(f"a captured step serves 1..{MAX_DECODE_ROWS} rows")
        _refuse_adaptive(layers)
        for i, layer in enumerate(layers):
            if not _device_only(layer):
                raise ValueError(f"layer {i} needs the host LRU (attach a device LRU to its pool)")
        hidden, top_k = layers[0].hidden, layers[0].top_k
        if any(layer.hidden != hidden or layer.top_k != top_k for layer in layers):
            raise ValueError("every layer of a step must have the same hidden size and top_k")
        device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.layers = layers
        self.x = torch.zeros((len(layers), rows, hidden), dtype=dtype, device=device)
        self.out = torch.zeros_like(self.x)
        self.inds = torch.zeros((len(layers), rows, top_k), dtype=torch.int32, device=device)
        self.scores = torch.zeros((len(layers), rows, top_k), dtype=dtype, device=device)
        self._args = []
        self._calls = []
        self._lrus = []      # (pool, the DeviceLru whose buffers the calls point at)
        lib = _lib.lib()
        for i, layer in enumerate(layers):
            a = layer.layer_args(self.x[i], self.out[i], self.inds[i], self.scores[i])
            sw = layer.switch_mlp
            lru = sw.pool.device_lru if sw.pool is not None else None
            if lru is not None:
                if rows * top_k > lru.usable_slots:
                    raise ValueError("requested experts exceed expert pool capacity")
                view = lru.view(sw.layer_id)
                self._lrus.append((sw.pool, lru))
                self._calls.append((lib.vm_moe_layer_lru, (ctypes.byref(a), ctypes.byref(view)), view))
            else:
                self._calls.append((lib.vm_moe_layer, (ctypes.byref(a),), None))
            self._args.append(a)
        self.stream = torch.cuda.Stream(device=device)
        self.graph = None

    def _check_state(self) -> None:
        _refuse_adaptive(self.layers)
        for pool, lru in self._lrus:
            if pool.device_lru is not lru:
                raise RuntimeError("a pool's device LRU was detached since the step was built")

    def _issue(self, handle) -> None:
        self._check_state()
        for fn, refs, _view in self._calls:
            _lib.check(fn(*refs, handle))

    def run_eager(self) -> torch.Tensor:
        """The step's calls launched one by one on the current stream."""
        self._issue(stream_handle())
        return self.out

    def capture(self) -> "StepGraph":
        """Record the step (nothing runs until ``replay``)."""
        graph = torch.cuda.CUDAGraph()
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.graph(graph, stream=self.stream, capture_error_mode="relaxed"):
            self._issue(stream_handle(torch.cuda.current_stream()))
        self.graph = graph
        return self

    def replay(self, x: torch.Tensor = None) -> torch.Tensor:
        """Launch the recorded step on the current stream, after copying ``x``
        [layers, rows, hidden] into the static inputs when given."""
        if self.graph is None:
            raise RuntimeError("capture() the step first")
        self._check_state()
        if x is not None:
            self.x.copy_(x)
        self.graph.replay()
        return self.out


__all__ = ["StepGraph"]
