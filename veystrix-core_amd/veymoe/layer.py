"""The MoE layer and its expert block on the gfx950 kernels.

``MoELayer.__call__(x)`` keeps the call signature and semantics of the
reference's patched ``Qwen3_5MoeSparseMoeBlock.__call__`` = ``_moe_call``
(models/flashnext/adaptive_topk.py:54-293) at its default threshold 1.0:

    gates  = softmax(gate(x), precise=True); inds = top-k; scores = renorm
    shared = shared_expert(x); shared_gate = sigmoid(shared_expert_gate(x))
    rows <= 8:  y = switch_mlp(x, inds, scores=scores, shared_y=shared_gate*shared)
    rows  > 8:  y = (switch_mlp(x, inds) * scores[..., None]).sum(-2) + shared_gate*shared

The decode branch runs as one C call (``vm_moe_layer``): router kernel (with
the shared gate), gate/up/SwiGLU kernel (routed + shared expert), down +
combine kernel.  Routed experts are dense arrays or an ``ExpertPool`` read
through a per-layer slot table on the device; when the pool does not hold
every routed expert, the call is split (router, host LRU assign + miss
staging, experts) exactly where the reference syncs routes to the host
(expert_cache.py:1738-1749, 1842-1947).

``HipSwitchGLU`` mirrors ``StreamingSwitchGLU.__call__(x, indices, allow_sort,
scores, shared_y, shared, shared_gate)`` (expert_cache.py:1709-1772): it
returns ``[..., hidden]`` when it combined (and sets ``_last_fused_shared``)
and ``[..., top_k, hidden]`` otherwise.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib, adaptive
from .device import act_code, ptr, q4proj, require_device, stream_handle
from .executor import HipMoEExecutor, Q4G32Projection, _as_projection
from .layout import RecordLayout
from .pool import ExpertPool, HostRecordStore

MAX_DECODE_ROWS = 8  # the reference's custom-combine bound (adaptive_topk.py:271-274)


@dataclass
class RouterLinear:
    """The router ``gate``: an unquantized bf16 Linear without bias ([E, H]).
    ``bias`` is an optional fp32 logit bias (synthetic popularity skew)."""
    weight: torch.Tensor
    bias: Optional[torch.Tensor] = None


@dataclass
class QuantizedMLP:
    """The shared expert: Q4/G32 gate/up/down projections, each [1, out, in/8]."""
    gate_proj: Q4G32Projection
    up_proj: Q4G32Projection
    down_proj: Q4G32Projection

    @property
    def inter(self) -> int:
        return int(self.gate_proj.weight.shape[-2])


class HipSwitchGLU:
    """Routed experts: dense expert-major projections or an HBM expert pool."""

    def __init__(self, hidden: int, inter: int, experts: int, *, projections=None, pool: ExpertPool = None,
                 layer_id: int = 0, host_store: HostRecordStore = None, group_size: int = 32):
        if (projections is None) == (pool is None):
            raise ValueError("give dense projections or an expert pool, not both")
        self.hidden = int(hidden)
        self.inter = int(inter)
        self.num_experts = int(experts)
        self.layer_id = int(layer_id)
        self.group_size = int(group_size)
        self.layout = RecordLayout(self.hidden, self.inter, self.group_size)
        self.pool = pool
        self.host_store = host_store
        if projections is not None:
            self.gate_proj = _as_projection(projections["gate_proj"])
            self.up_proj = _as_projection(projections["up_proj"])
            self.down_proj = _as_projection(projections["down_proj"])
        else:
            self.gate_proj = self.up_proj = self.down_proj = None
        self._executor = None
        self._last_fused_shared = False
        self.hits = 0
        self.misses = 0

    @property
    def metal_combines_scores(self) -> bool:
        """Name kept from the reference: the patched MoE block asks it whether the
        expert block combines scores itself (expert_cache.py:1434-1443).  As
        there, layer 0 does not: its decode rows go through the generic combine
        ``(y * scores[..., None]).sum(-2) + shared`` (adaptive_topk.py:271-278)."""
        return self.layer_id > 0

    def executor(self, top_k: int) -> HipMoEExecutor:
        if self._executor is None or self._executor.top_k != top_k:
            self._executor = HipMoEExecutor(max(self.num_experts, top_k), self.hidden, top_k)
        return self._executor

    # ------------------------------------------------------------- pool ---
    def _pool_fully_resident(self) -> bool:
        """True when no call can change the pool's LRU state in a way that
        matters: every expert of this layer is resident and the pool holds
        every key of every layer, so nothing is ever evicted.  Otherwise a
        call must make the host LRU pass even when all its experts hit, since
        the reference moves hits to the most recent end (expert_pool.py:
        139-144) and that order decides later evictions."""
        pool = self.pool
        table = pool._host_table[self.layer_id]
        return bool((table >= 0).all()) and pool.holds_every_key()

    def resolve_routes(self, routed) -> np.ndarray:
        """Host LRU pass for a pool-backed layer: assign, stage misses, and
        return route words ``SLOT_BIT | slot`` (expert_cache.py:1842-1917)."""
        pool = self.pool
        wanted = list(dict.fromkeys(int(e) for e in routed))
        slots, misses = pool.assign(self.layer_id, wanted)
        self.hits += len(routed) - len(misses)
        self.misses += len(misses)
        if misses:
            if self.host_store is None:
                pool.invalidate(self.layer_id, misses)
                raise RuntimeError("expert pool miss with no host record store to fill from")
            pool.fill(self.layer_id, misses, self.host_store)
        return np.array([0x80000000 | slots[int(e)] for e in routed], dtype=np.uint32)

    def _dense_or_pool_args(self):
        if self.pool is not None:
            return (None, None, None), self.pool.view()
        return (self.gate_proj, self.up_proj, self.down_proj), _lib.VmPoolView()

    def __call__(self, x, indices, allow_sort=True, scores=None, shared_y=None, shared=None, shared_gate=None):
        self._last_fused_shared = False
        hidden = x.shape[-1]
        flat = x.reshape(-1, hidden).contiguous()
        k = int(indices.shape[-1])
        flat_inds = indices.reshape(-1, k).to(torch.int32).contiguous()
        rows = flat.shape[0]
        if rows > MAX_DECODE_ROWS and flat.dtype == torch.bfloat16:
            # the reference's rows > 8 path: per-slot expert outputs
            # (expert_cache.py:1949-2037).  grouped_experts makes the call's
            # only LRU pass over a pool, so hits and misses count once.
            from .grouped import grouped_experts

            return grouped_experts(self, flat, flat_inds).reshape(*x.shape[:-1], k, hidden)
        executor = self.executor(k)
        executor.max_tokens = max(executor.max_tokens, 1)
        if self.pool is not None:
            routed = flat_inds.reshape(-1).tolist()  # route sync (expert_cache.py:1738-1749)
            words = self.resolve_routes(routed)
            routes = torch.from_numpy(words.view(np.int32).reshape(rows, k)).to(flat.device)
            projections = self._pool_placeholders(flat.device)
            slab = self.pool
        else:
            routes = flat_inds
            projections = (self.gate_proj, self.up_proj, self.down_proj)
            slab = None
        # the custom (combining) path only where the reference takes it:
        # scores given, rows <= 8 and metal_combines_scores (expert_cache.py:1763-1767)
        combine = scores is not None and rows <= MAX_DECODE_ROWS and self.metal_combines_scores
        if combine:
            out = executor._run(flat, routes, *projections, self.inter, False,
                                scores.reshape(rows, k).contiguous(), slab, None,
                                shared_y, shared, shared_gate, None)
            if shared_y is not None or (shared is not None and shared_gate is not None):
                self._last_fused_shared = True
            return out.reshape(*x.shape[:-1], hidden)
        out = executor._run(flat, routes, *projections, self.inter, False, None, slab, None, None, None, None,
                            None)
        return out.reshape(*x.shape[:-1], k, hidden)

    def _pool_placeholders(self, device):
        """Zero-size dense projections for pool-only calls (shape checks only)."""
        empty_w = torch.empty((0, self.inter, self.hidden // 8), dtype=torch.int32, device=device)
        empty_m = torch.empty((0, self.inter, self.hidden // self.group_size), dtype=torch.bfloat16,
                              device=device)
        empty_dw = torch.empty((0, self.hidden, self.inter // 8), dtype=torch.int32, device=device)
        empty_dm = torch.empty((0, self.hidden, self.inter // self.group_size), dtype=torch.bfloat16,
                               device=device)
        return (_NullProj(empty_w, empty_m, empty_m), _NullProj(empty_w, empty_m, empty_m),
                _NullProj(empty_dw, empty_dm, empty_dm))


class _NullProj(Q4G32Projection):
    """A projection whose pointers are passed as NULL (pool-addressed experts)."""


class MoELayer:
    """One SwiGLU MoE layer: router, routed experts, shared expert, combine."""

    def __init__(self, gate: RouterLinear, switch_mlp: HipSwitchGLU, top_k: int, *,
                 shared_expert: QuantizedMLP = None, shared_expert_gate: Q4G32Projection = None,
                 layer_id: int = None, renorm_blend: float = 1.0):
        if (shared_expert is None) != (shared_expert_gate is None):
            raise ValueError("shared_expert and shared_expert_gate go together")
        self.gate = gate
        self.switch_mlp = switch_mlp
        self.top_k = int(top_k)
        self.shared_expert = shared_expert
        self.shared_expert_gate = shared_expert_gate
        self._flashnext_layer_id = switch_mlp.layer_id if layer_id is None else layer_id
        self.renorm_blend = float(renorm_blend)
        self.last_inds = None
        self.last_scores = None
        self._ws = {}
        self._args_cache = {}
        self._route_host = None   # pinned host copy of the routed ids (split-phase path)
        self._route_event = None

    @property
    def hidden(self) -> int:
        return self.switch_mlp.hidden

    # --------------------------------------------------------- decode ---
    def layer_args(self, x: torch.Tensor, out: torch.Tensor, inds: torch.Tensor = None,
                   scores: torch.Tensor = None) -> _lib.VmLayerArgs:
        """The C arguments of one decode call on fixed buffers (reusable)."""
        sw = self.switch_mlp
        tokens = x.shape[0]
        dtype = act_code(x)
        shared_inter = self.shared_expert.inter if self.shared_expert is not None else 0
        lib = _lib.lib()
        key = (tokens, dtype, x.device)
        ws = self._ws.get(key)
        if ws is None:
            nbytes = int(lib.vm_moe_layer_workspace(tokens, self.top_k, sw.hidden, sw.inter, shared_inter,
                                                    sw.num_experts, dtype))
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=x.device)
            self._ws[key] = ws
        a = _lib.VmLayerArgs()
        a.x = ptr(x)
        a.output = ptr(out)
        a.router_weight = ptr(self.gate.weight)
        a.router_bias = ptr(self.gate.bias)
        if sw.pool is not None:
            a.pool = sw.pool.view()
            a.slot_table = ptr(sw.pool.table(sw.layer_id))
        else:
            a.gate = q4proj(sw.gate_proj.weight, sw.gate_proj.scales, sw.gate_proj.biases)
            a.up = q4proj(sw.up_proj.weight, sw.up_proj.scales, sw.up_proj.biases)
            a.down = q4proj(sw.down_proj.weight, sw.down_proj.scales, sw.down_proj.biases)
        if self.shared_expert is not None:
            se = self.shared_expert
            a.shared_gate_proj = q4proj(se.gate_proj.weight, se.gate_proj.scales, se.gate_proj.biases)
            a.shared_up_proj = q4proj(se.up_proj.weight, se.up_proj.scales, se.up_proj.biases)
            a.shared_down_proj = q4proj(se.down_proj.weight, se.down_proj.scales, se.down_proj.biases)
            g = self.shared_expert_gate
            a.shared_expert_gate = q4proj(g.weight, g.scales, g.biases)
        a.inds_out = ptr(inds)
        a.scores_out = ptr(scores)
        a.workspace = ptr(ws)
        a.workspace_bytes = ws.numel()
        a.tokens, a.hidden_size, a.inter_size = tokens, sw.hidden, sw.inter
        a.shared_inter = shared_inter
        a.expert_count, a.top_k, a.group_size = sw.num_experts, self.top_k, sw.group_size
        a.act_dtype = dtype
        a.renorm_blend = self.renorm_blend
        # layer 0 combines like the reference's generic path (expert_cache.py:1434-1443)
        a.combine = _lib.VM_COMBINE_FUSED if sw.metal_combines_scores else _lib.VM_COMBINE_GENERIC
        return a

    def forward(self, flat: torch.Tensor, inject=None) -> torch.Tensor:
        """The layer on [rows, hidden]: rows <= 8 run the fused decode kernels,
        more rows the grouped path (router GEMM, device token-by-expert sort,
        MFMA grouped experts, generic combine); both inside vm_moe_layer.

        ``inject = (streams [rows, hc*hidden], weights [rows, hc], out)``: the
        experts' final epilogue also writes the hyper-connection injection of
        the layer output into the residual streams (compile_glue.py:32-35)
        into ``out`` (which may be ``streams``)."""
        require_device("x", flat, (torch.bfloat16, torch.float32))
        tokens = flat.shape[0]
        out = torch.empty_like(flat)
        # the C arguments are built once per (rows, dtype, device); a call only
        # patches the activation pointers (inds/scores live in per-layer buffers)
        key = (tokens, flat.dtype, flat.device)
        cached = self._args_cache.get(key)
        if cached is None:
            inds = torch.empty((tokens, self.top_k), dtype=torch.int32, device=flat.device)
            scores = torch.empty((tokens, self.top_k), dtype=flat.dtype, device=flat.device)
            cached = (self.layer_args(flat, out, inds, scores), inds, scores)
            self._args_cache[key] = cached
        args, inds, scores = cached
        args.x = ptr(flat)
        args.output = ptr(out)
        args.phases = 0
        self._set_inject(args, flat, inject)
        lib = _lib.lib()
        sw = self.switch_mlp
        layer = self._flashnext_layer_id
        exact = adaptive.threshold_for(layer) >= 1.0
        if exact:
            adaptive.record_exact(layer, tokens, self.top_k)
        lru = sw.pool.device_lru if sw.pool is not None else None
        if lru is not None:
            if tokens > MAX_DECODE_ROWS or not exact or adaptive.observing():
                # the grouped path and the adaptive plan resolve their
                # experts on the host: hand the LRU state back for this call,
                # then upload it into the same device buffers (a sync and an
                # O(slots) host pass each way)
                sw.pool.detach_device_lru()
                try:
                    return self._forward_host(args, inds, scores, flat, out, exact)
                finally:
                    sw.pool.attach_device_lru(lru.store, reuse=lru)
            if tokens * self.top_k > lru.usable_slots:
                raise ValueError("requested experts exceed expert pool capacity")
            # router, assign, fill and experts on the device: no route sync
            _lib.check(lib.vm_moe_layer_lru(args, lru.view(sw.layer_id), stream_handle()))
            self.last_inds, self.last_scores = inds, scores
            return out
        return self._forward_host(args, inds, scores, flat, out, exact)

    def _forward_host(self, args, inds: torch.Tensor, scores: torch.Tensor, flat: torch.Tensor, out: torch.Tensor,
                      exact: bool) -> torch.Tensor:
        """The layer call whose routes the host may see: the adaptive plan or
        a route observer, or a pool whose LRU state is on the host."""
        lib = _lib.lib()
        sw = self.switch_mlp
        if not exact or adaptive.observing():
            return self._forward_adaptive(args, inds, scores, flat, out)
        if sw.pool is not None and not sw._pool_fully_resident():
            # router, then the host LRU pass on synced routes, then the experts
            args.phases = _lib.VM_PHASE_ROUTER
            _lib.check(lib.vm_moe_layer(args, stream_handle()))
            self._host_lru_pass(self._routes_to_host(inds))
            args.phases = _lib.VM_PHASE_EXPERTS
        _lib.check(lib.vm_moe_layer(args, stream_handle()))
        self.last_inds, self.last_scores = inds, scores
        return out

    def _host_lru_pass(self, routed: list) -> None:
        """assign() of the routed ids in first-seen order, staging the misses
        from the host record store (expert_cache.py:1842-1947)."""
        sw = self.switch_mlp
        wanted = list(dict.fromkeys(routed))
        slots, misses = sw.pool.assign(sw.layer_id, wanted)
        sw.hits += len(routed) - len(misses)
        sw.misses += len(misses)
        if misses:
            if sw.host_store is None:
                sw.pool.invalidate(sw.layer_id, misses)
                raise RuntimeError("expert pool miss with no host record store to fill from")
            sw.pool.fill(sw.layer_id, misses, sw.host_store)
        sw.pool.sync_tables()

    def _forward_adaptive(self, args, inds: torch.Tensor, scores: torch.Tensor, flat: torch.Tensor,
                          out: torch.Tensor) -> torch.Tensor:
        """A threshold below 1.0 (adaptive_topk.py:76-262): a router-only call
        that also writes the gates, the host plan of ``veymoe.adaptive``, the
        pool's host LRU pass on the planned routes, and an experts-only call
        on them.  The experts call keeps all top_k slots: dropped slots route
        to the row's first expert with score 0 and add nothing.  At threshold
        1.0 with a route observer set, the observer sees the routes and they
        stay as selected (adaptive_topk.py:240-253)."""
        lib = _lib.lib()
        sw = self.switch_mlp
        gates = torch.empty((flat.shape[0], sw.num_experts), dtype=flat.dtype, device=flat.device)
        args.phases = _lib.VM_PHASE_ROUTER
        args.gates_out = ptr(gates)
        try:
            _lib.check(lib.vm_moe_layer(args, stream_handle()))
        finally:
            args.gates_out = None
        picked = torch.gather(gates, 1, inds.long()).float().cpu().numpy()
        host_inds = inds.cpu().numpy()
        layer = self._flashnext_layer_id
        if adaptive.threshold_for(layer) >= 1.0:
            # exact routing with a route observer: it sees the routes, which stay
            adaptive.observe_exact(layer, host_inds, picked)
            routed = host_inds.reshape(-1).tolist()
        else:
            new_inds, new_scores, _, width = adaptive.plan(layer, host_inds, picked, self.renorm_blend,
                                                           bf16=flat.dtype == torch.bfloat16)
            inds.copy_(torch.from_numpy(new_inds))
            scores.copy_(torch.from_numpy(new_scores).to(scores.dtype))
            # the routes the reference's expert block receives: cut to the width
            routed = new_inds[:, :width].reshape(-1).tolist()
        if sw.pool is not None and not sw._pool_fully_resident():
            self._host_lru_pass(routed)
        args.phases = _lib.VM_PHASE_EXPERTS
        _lib.check(lib.vm_moe_layer(args, stream_handle()))
        self.last_inds, self.last_scores = inds, scores
        return out

    @staticmethod
    def _set_inject(args, flat: torch.Tensor, inject) -> None:
        if inject is None:
            args.inject_hidden = args.inject_weights = args.inject_out = None
            args.hc_count = 0
            return
        streams, weights, target = inject
        rows = flat.shape[0]
        for name, t in (("streams", streams), ("weights", weights), ("out", target)):
            require_device(name, t, (flat.dtype,))
            if not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous")
        hc = weights.shape[-1]
        if weights.numel() != rows * hc or streams.numel() != rows * hc * flat.shape[1] or \
                target.numel() != streams.numel():
            raise ValueError("injection shapes must be streams [rows, hc*hidden], weights [rows, hc]")
        args.inject_hidden = ptr(streams)
        args.inject_weights = ptr(weights)
        args.inject_out = ptr(target)
        args.hc_count = hc

    def _routes_to_host(self, inds: torch.Tensor) -> list:
        """The routed expert ids on the host: one D2H copy into a pinned
        buffer kept per layer, then a wait on its event."""
        n = inds.numel()
        host = self._route_host
        if host is None or host.numel() != n:
            host = self._route_host = torch.empty(n, dtype=torch.int32, pin_memory=True)
            self._route_event = torch.cuda.Event()
        host.copy_(inds.reshape(-1), non_blocking=True)
        self._route_event.record()
        self._route_event.synchronize()
        return host.tolist()

    decode = forward
    prefill = forward

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        hidden = x.shape[-1]
        flat = x.reshape(-1, hidden).contiguous()
        return self.forward(flat).reshape(x.shape)
