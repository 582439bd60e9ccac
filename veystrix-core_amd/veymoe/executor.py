"""Bounded three-projection MoE executor on hand-written gfx950 kernels.

Drop-in counterpart of the reference's ``MetalMoEExecutor``
(models/flashnext/metal_runtime.py:427-974): same constructor bounds, same
``execute`` keywords and shape contract (ValueError/TypeError texts of
:446-461 and :837-895), ``weighted_combine`` (:145-191) and
``probe_capabilities`` (:65-96).  Differences, deliberate:

* tensors are torch tensors on the GPU (bf16 or fp32 activations, uint32/int32
  packed weights, bf16 scales and biases);
* there is no reference fallback: when the HIP library or a gfx950 device is
  missing, ``execute`` raises ``RuntimeError`` after validating its arguments
  (the reference would silently compute on the CPU);
* ``slab_pack`` is an ``ExpertPool`` or a device byte buffer of records in
  ``RecordLayout(hidden, inter)``; the reference requires 2560/640;
* gate/up/SwiGLU always run fused (one kernel); ``fused_up_swiglu`` is kept
  for the API and its values give identical results.
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any, Mapping, Sequence

import numpy as np

from . import _lib

MAX_TOKENS = 8
MAX_EXPERTS = 512
MAX_TOP_K = 10
MAX_WIDTH = 16_384
GROUP_SIZE = 32
SUPPORTED_GROUP_SIZES = (32,)
BITS = 4


@dataclass(frozen=True)
class Q4G32Projection:
    """Packed expert rows consumed by one gate, up, or down projection."""

    weight: Any
    scales: Any
    biases: Any


@dataclass(frozen=True)
class HipCapabilities:
    available: bool
    supports_custom_moe: bool
    backend: str
    reason: str

    @property
    def custom_hip(self) -> bool:
        return self.supports_custom_moe

    def __getitem__(self, key: str) -> Any:
        return getattr(self, key)


def probe_capabilities(backend: Any = None) -> HipCapabilities:
    """Capability flags without launching a kernel.

    ``backend`` may be ``"hip"``, ``"reference"`` or an object exposing
    ``available``/``supports_custom_moe`` (injected in host-only tests)."""
    if backend == "reference":
        return HipCapabilities(False, False, "reference", "reference backend requested")
    if backend is not None and hasattr(backend, "available"):
        available = bool(getattr(backend, "available"))
        supports = bool(getattr(backend, "supports_custom_moe", False))
        reason = "injected backend capability"
        if not available:
            reason = "injected backend is unavailable"
        elif not supports:
            reason = "backend does not provide custom MoE"
        return HipCapabilities(available and supports, supports, "injected", reason)
    if backend not in (None, "hip"):
        return HipCapabilities(False, False, str(backend), "unknown backend")
    try:
        lib = _lib.lib()
    except _lib.ExtensionMissing as exc:
        return HipCapabilities(False, False, "hip", str(exc))
    try:
        import torch

        if not torch.cuda.is_available():
            return HipCapabilities(False, False, "hip", "no GPU is visible to torch")
    except Exception as exc:  # pragma: no cover - environment dependent
        return HipCapabilities(False, False, "hip", f"torch unavailable: {exc}")
    if not lib.vm_available():
        return HipCapabilities(False, False, "hip", _lib.last_error() or "device is not gfx950")
    return HipCapabilities(True, True, "hip", "gfx950 device detected")


def _as_projection(value: Any) -> Q4G32Projection:
    if isinstance(value, Q4G32Projection):
        return value
    if isinstance(value, Mapping):
        return Q4G32Projection(value["weight"], value["scales"], value["biases"])
    if isinstance(value, Sequence) and len(value) == 3:
        return Q4G32Projection(value[0], value[1], value[2])
    raise TypeError("projection must be (weight, scales, biases)")


def _shape(value: Any) -> tuple[int, ...]:
    return tuple(int(item) for item in value.shape)


def _is_word_dtype(dtype) -> bool:
    name = str(dtype)
    return name in ("torch.int32", "torch.uint32", "uint32", "int32") or (
        isinstance(dtype, np.dtype) and dtype in (np.uint32, np.int32))


def _validate_projection(projection: Q4G32Projection, expert_count: int | None, input_width: int,
                         output_width: int, group_size: int = GROUP_SIZE) -> None:
    weight_shape = _shape(projection.weight)
    scale_shape = _shape(projection.scales)
    bias_shape = _shape(projection.biases)
    count = weight_shape[0] if expert_count is None else expert_count
    expected_weight = (count, output_width, input_width // 8)
    expected_meta = (count, output_width, input_width // group_size)
    if weight_shape != expected_weight:
        raise ValueError(f"weight shape {weight_shape} != {expected_weight}")
    if scale_shape != expected_meta or bias_shape != expected_meta:
        raise ValueError(f"Q4/G{group_size} scales and biases have an invalid shape")
    if not _is_word_dtype(getattr(projection.weight, "dtype", None)):
        raise TypeError("Q4 weights must use uint32 packed values")


def weighted_combine(expert_outputs: Any, routes: Any, scores: Any) -> Any:
    """Combine routed expert outputs with the router scores (GPU).

    Normal form ``expert_outputs[..., slots, hidden]``; when the outputs hold
    every expert ``[..., experts, hidden]``, ``routes`` selects the slots
    first.  The sum is accumulated in fp32 in slot order."""
    output_shape = _shape(expert_outputs)
    route_shape = _shape(routes)
    score_shape = _shape(scores)
    if len(output_shape) < 2 or len(route_shape) == 0:
        raise ValueError("expert_outputs and routes need at least one dimension")
    if score_shape != route_shape:
        raise ValueError("routes and scores must have identical shapes")
    slots = route_shape[-1]
    import torch

    from .device import act_code, ptr, require_device, stream_handle

    if output_shape[:-1] == route_shape:
        selected = expert_outputs
    elif len(output_shape) == len(route_shape) + 1 and output_shape[-2] >= slots:
        if isinstance(routes, np.ndarray) and routes.size and (
                routes.min() < 0 or routes.max() >= output_shape[-2]):
            raise ValueError("routes contain an expert outside expert_outputs")
        require_device("routes", routes)
        selected = torch.take_along_dim(expert_outputs, routes.long().unsqueeze(-1), dim=-2)
    else:
        raise ValueError(f"expert_outputs shape {output_shape} does not match routes {route_shape}")
    if _shape(selected)[:-1] != route_shape:
        raise ValueError("selected expert outputs do not match route slots")
    selected = require_device("expert_outputs", selected.contiguous())
    require_device("scores", scores, (torch.bfloat16, torch.float32))
    hidden = output_shape[-1]
    tokens = int(np.prod(route_shape[:-1], dtype=np.int64)) if len(route_shape) > 1 else 1
    out = torch.empty((*route_shape[:-1], hidden), dtype=selected.dtype, device=selected.device)
    rc = _lib.lib().vm_weighted_combine(ptr(selected), ptr(scores.contiguous()), ptr(out), tokens, slots, hidden,
                                        act_code(selected), act_code(scores), stream_handle())
    _lib.check(rc)
    return out


def _pool_view(pack, layout, header_size: int, with_header: bool = True):
    """VmPoolView of an ExpertPool or a raw device byte buffer."""
    from .pool import ExpertPool

    if pack is None:
        return _lib.VmPoolView()
    if isinstance(pack, ExpertPool):
        if pack.layout.hidden != layout.hidden or pack.layout.inter != layout.inter:
            raise ValueError("expert pool layout does not match the executor shapes")
        return pack.view()
    from .device import require_device

    require_device("slab_pack", pack)
    header = header_size if with_header else 0
    nbytes = pack.numel() * pack.element_size()
    view = _lib.VmPoolView()
    view.base = pack.data_ptr()
    view.header_size = header
    view.record_stride = layout.record_stride
    for i, offset in enumerate(layout.part_offsets()):
        view.part_offset[i] = offset
    view.records = max(0, (nbytes - header) // layout.record_stride)
    return view


class HipMoEExecutor:
    """Bounded three-projection executor on the gfx950 kernels."""

    def __init__(self, expert_count: int, hidden_size: int, top_k: int, backend: Any = None, *,
                 max_tokens: int = MAX_TOKENS, max_width: int = MAX_WIDTH,
                 profile_boundaries: bool | None = None, profile_boundary: str | None = None,
                 fused_up_swiglu: bool | None = None, group_size: int = GROUP_SIZE,
                 header_size: int = 4096, fma_dequant: bool | None = None) -> None:
        if not 1 <= expert_count <= MAX_EXPERTS:
            raise ValueError(f"expert_count must be in 1..{MAX_EXPERTS}")
        if hidden_size <= 0:
            raise ValueError("hidden_size must be positive")
        if not 1 <= top_k <= MAX_TOP_K:
            raise ValueError(f"top_k must be in 1..{MAX_TOP_K}")
        if top_k > expert_count:
            raise ValueError("top_k cannot exceed expert_count")
        if not 1 <= max_tokens <= MAX_TOKENS:
            raise ValueError(f"max_tokens must be in 1..{MAX_TOKENS}")
        if not 1 <= max_width <= MAX_WIDTH:
            raise ValueError(f"max_width must be in 1..{MAX_WIDTH}")
        if group_size not in SUPPORTED_GROUP_SIZES:
            raise ValueError(f"group_size must be one of {SUPPORTED_GROUP_SIZES}")
        self.expert_count = int(expert_count)
        self.hidden_size = int(hidden_size)
        self.top_k = int(top_k)
        self.max_tokens = int(max_tokens)
        self.max_width = int(max_width)
        self.group_size = int(group_size)
        self.header_size = int(header_size)
        self.fma_dequant = bool(fma_dequant)
        self.backend = backend
        self.capabilities = probe_capabilities(backend)
        self.last_path = "none"
        self.fallback_reason = self.capabilities["reason"]
        if fused_up_swiglu is None:
            fused_up_swiglu = os.environ.get("FLASHNEXT_FUSED_UP_SWIGLU") == "1"
        self.fused_up_swiglu = bool(fused_up_swiglu)
        self._status = None

    @property
    def available(self) -> bool:
        return bool(self.capabilities["available"])

    def _require(self):
        if not self.capabilities.supports_custom_moe or not self.available:
            raise RuntimeError(f"custom MoE is unavailable on this backend: {self.capabilities.reason}")

    # ------------------------------------------------------------------
    def status(self, reset: bool = True) -> int:
        """Bit 0 set when a route or slot was out of range since the last reset."""
        if self._status is None:
            return 0
        value = int(self._status.item())
        if reset:
            self._status.zero_()
        return value

    def _status_ptr(self, device):
        import torch

        if self._status is None:
            self._status = torch.zeros(1, dtype=torch.int32, device=device)
        return self._status.data_ptr()

    def execute(self, x: Any, routes: Any, projections: Mapping[str, Any] | Sequence[Any] | Any = None, *,
                return_all: bool = False, scores: Any = None, slab_pack: Any = None, stream_pack: Any = None,
                shared_y: Any = None, shared: Any = None, shared_gate: Any = None,
                pool_activation: Any = None) -> Any:
        """Run gate, up, activation and down for bounded flattened inputs.

        ``x`` is ``(tokens, hidden_size)``, ``routes`` ``(tokens, top_k)`` route
        words; projections map ``gate_proj/up_proj/down_proj`` to
        (weight, scales, biases) or are a three-item sequence."""
        # combine-only forms (metal_runtime.py:820-835)
        if projections is not None and not isinstance(projections, (Mapping, list, tuple)):
            self._require()
            self.last_path = "hip"
            self.fallback_reason = None
            return weighted_combine(x, routes, projections)
        if projections is None and scores is not None:
            self._require()
            self.last_path = "hip"
            self.fallback_reason = None
            return weighted_combine(x, routes, scores)
        if projections is None:
            raise TypeError("packed execution needs gate, up, and down projections")
        x_shape = _shape(x)
        route_shape = _shape(routes)
        if len(x_shape) != 2 or x_shape[1] != self.hidden_size:
            raise ValueError("x must have shape (tokens, hidden_size)")
        if len(route_shape) != 2 or route_shape[1] != self.top_k:
            raise ValueError("routes must have shape (tokens, top_k)")
        if scores is not None and _shape(scores) != route_shape:
            raise ValueError("scores must have the same shape as routes")
        if (shared is None) != (shared_gate is None):
            raise ValueError("shared and shared_gate must be provided together")
        if shared_y is not None and shared is not None:
            raise ValueError("provide shared_y or shared parts, not both")
        if stream_pack is not None and slab_pack is None:
            raise ValueError("stream pack requires a resident slab pack")
        tokens = x_shape[0]
        if route_shape[0] != tokens:
            raise ValueError("x and routes must have the same token count")
        if not 1 <= tokens <= self.max_tokens:
            raise ValueError(f"tokens must be in 1..{self.max_tokens}")
        if isinstance(routes, np.ndarray) and np.any(routes < 0):
            raise ValueError("routes contain an expert outside the configured bank")
        if isinstance(projections, Mapping):
            gate = _as_projection(projections["gate_proj"])
            up = _as_projection(projections["up_proj"])
            down = _as_projection(projections["down_proj"])
        else:
            if len(projections) != 3:
                raise ValueError("projections must contain gate, up, and down")
            gate, up, down = (_as_projection(item) for item in projections)
        gate_width = _shape(gate.weight)[1]
        inter_width = _shape(up.weight)[1]
        if gate_width != inter_width or gate_width > self.max_width:
            raise ValueError("gate and up projection widths must match the bound")
        _validate_projection(gate, None, self.hidden_size, gate_width, self.group_size)
        _validate_projection(up, None, self.hidden_size, inter_width, self.group_size)
        if self.hidden_size % self.group_size or inter_width % self.group_size:
            raise ValueError(f"Q4/G{self.group_size} projection inputs must be group aligned")
        _validate_projection(down, None, inter_width, self.hidden_size, self.group_size)
        if pool_activation is not None:
            if (slab_pack is None or stream_pack is not None or return_all
                    or _shape(pool_activation) != (*route_shape, inter_width)):
                raise ValueError("invalid precomputed pool activation")
        self._require()
        return self._run(x, routes, gate, up, down, inter_width, return_all, scores, slab_pack, stream_pack,
                         shared_y, shared, shared_gate, pool_activation)

    def _run(self, x, routes, gate, up, down, inter, return_all, scores, slab_pack, stream_pack, shared_y,
             shared, shared_gate, pool_activation, activations_only=False):
        import torch

        from .device import act_code, ptr, q4proj, require_device, stream_handle, word_tensor
        from .layout import RecordLayout

        require_device("x", x, (torch.bfloat16, torch.float32))
        word_tensor("routes", routes)
        for proj in (gate, up, down):
            word_tensor("weight", proj.weight)
            require_device("scales", proj.scales, (torch.bfloat16,))
            require_device("biases", proj.biases, (torch.bfloat16,))
        tokens, slots = _shape(routes)
        dtype = x.dtype
        layout = RecordLayout(self.hidden_size, inter, self.group_size)
        args = _lib.VmMoeArgs()
        args.x = ptr(x)
        args.gate = q4proj(gate.weight, gate.scales, gate.biases)
        args.up = q4proj(up.weight, up.scales, up.biases)
        args.down = q4proj(down.weight, down.scales, down.biases)
        args.pool = _pool_view(slab_pack, layout, self.header_size)
        args.stream = _pool_view(stream_pack, layout, 0, with_header=False)
        args.routes = ptr(routes)
        if scores is not None and not return_all:
            require_device("scores", scores, (torch.bfloat16, torch.float32))
            args.scores = ptr(scores)
            args.score_dtype = act_code(scores)
            if shared_y is not None:
                shared_y = require_device("shared_y", shared_y.reshape(tokens, self.hidden_size).to(dtype))
                args.shared_y = ptr(shared_y)
            elif shared is not None:
                shared = require_device("shared", shared.reshape(tokens, self.hidden_size).to(dtype))
                shared_gate = require_device("shared_gate", shared_gate.reshape(tokens).to(dtype).contiguous())
                args.shared = ptr(shared)
                args.shared_gate = ptr(shared_gate)
        gate_out = up_out = None
        if return_all:
            gate_out = torch.empty((tokens, slots, inter), dtype=dtype, device=x.device)
            up_out = torch.empty_like(gate_out)
            args.gate_out = ptr(gate_out)
            args.up_out = ptr(up_out)
        act_out = None
        if pool_activation is not None:
            pool_activation = require_device("pool_activation", pool_activation.to(dtype).contiguous())
            args.activation_in = ptr(pool_activation)
        elif activations_only:
            act_out = torch.empty((tokens, slots, inter), dtype=dtype, device=x.device)
            args.activation_out = ptr(act_out)
        if activations_only:
            out = None
        elif args.scores:
            out = torch.empty((tokens, self.hidden_size), dtype=dtype, device=x.device)
        else:
            out = torch.empty((tokens, slots, self.hidden_size), dtype=dtype, device=x.device)
        args.output = ptr(out)
        ws = torch.empty(int(_lib.lib().vm_moe_execute_workspace(tokens, slots, inter, act_code(x))),
                         dtype=torch.uint8, device=x.device)
        args.workspace = ptr(ws)
        args.workspace_bytes = ws.numel()
        args.status = self._status_ptr(x.device)
        args.tokens, args.slots = tokens, slots
        args.hidden_size, args.inter_size = self.hidden_size, inter
        dense_count = _shape(gate.weight)[0]
        args.expert_count = dense_count if dense_count > 0 else self.expert_count
        args.group_size = self.group_size
        args.act_dtype = act_code(x)
        _lib.check(_lib.lib().vm_moe_execute(args, stream_handle()))
        self.last_path = "hip"
        self.fallback_reason = None
        if activations_only:
            return act_out
        if return_all:
            return gate_out, up_out, out
        return out

    def pool_activations(self, x, routes, projections, slab_pack):
        """Per-route SwiGLU activations [T, k, I] (gate and up only)."""
        gate, up = (_as_projection(projection) for projection in projections[:2])
        down = _as_projection(projections[2])
        self._require()
        width = _shape(up.weight)[1]
        return self._run(x, routes, gate, up, down, width, False, None, slab_pack, None, None, None, None, None,
                         activations_only=True)

    def affine_singleton(self, x, weight, scales, biases):
        """Project one row through one unpacked Q4 expert: returns [1, out]."""
        import torch

        self._require()
        proj = Q4G32Projection(weight[None], scales[None], biases[None])
        routes = torch.zeros((1, 1), dtype=torch.int32, device=x.device)
        out_width = _shape(weight)[0]
        saved = self.top_k
        try:
            self.top_k = 1
            down = Q4G32Projection(
                torch.zeros((1, self.hidden_size, out_width // 8), dtype=torch.int32, device=x.device),
                torch.zeros((1, self.hidden_size, out_width // self.group_size), dtype=torch.bfloat16,
                            device=x.device),
                torch.zeros((1, self.hidden_size, out_width // self.group_size), dtype=torch.bfloat16,
                            device=x.device))
            gate_out, _, _ = self._run(x, routes, proj, proj, down, out_width, True, None, None, None, None,
                                       None, None, None)
        finally:
            self.top_k = saved
        return gate_out[:, 0, :]


__all__ = [
    "BITS", "GROUP_SIZE", "MAX_EXPERTS", "MAX_TOKENS", "MAX_TOP_K", "MAX_WIDTH", "HipCapabilities",
    "HipMoEExecutor", "Q4G32Projection", "SUPPORTED_GROUP_SIZES", "probe_capabilities", "weighted_combine",
]
