"""Router softmax / top-k / renormalisation on the GPU.

Counterpart of ``_router_plain`` + ``_renorm_plain`` (models/flashnext/compiled.py:61-71)
and the router lines of ``_moe_call`` (adaptive_topk.py:59-65, 257-262):
``softmax(x @ W.T, precise=True)``, top-k, ``scores / (topk_mass + blend *
(selected_mass - topk_mass))``.  Tie rule (MLX's argpartition leaves it open):
gate descending, then expert index ascending; the selection comes back in
that order.
"""
from __future__ import annotations

import torch

from . import _lib
from .device import act_code, ptr, require_device, stream_handle


def router_topk(x: torch.Tensor, weight: torch.Tensor, top_k: int, *, logit_bias: torch.Tensor | None = None,
                renorm_blend: float = 1.0, return_gates: bool = False):
    """x [T, H] (bf16/fp32), weight [E, H] bf16 -> (inds int32 [T, k], scores [T, k][, gates [T, E]])."""
    require_device("x", x, (torch.bfloat16, torch.float32))
    require_device("weight", weight, (torch.bfloat16,))
    tokens, hidden = x.shape
    experts = weight.shape[0]
    if weight.shape[1] != hidden:
        raise ValueError("router weight must have shape (experts, hidden)")
    if logit_bias is not None:
        require_device("logit_bias", logit_bias, (torch.float32,))
    inds = torch.empty((tokens, top_k), dtype=torch.int32, device=x.device)
    scores = torch.empty((tokens, top_k), dtype=x.dtype, device=x.device)
    gates = torch.empty((tokens, experts), dtype=x.dtype, device=x.device) if return_gates else None
    lib = _lib.lib()
    ws = torch.zeros(int(lib.vm_router_workspace(tokens, experts)), dtype=torch.uint8, device=x.device)
    args = _lib.VmRouterArgs()
    args.x = ptr(x)
    args.weight = ptr(weight)
    args.logit_bias = ptr(logit_bias)
    args.inds = ptr(inds)
    args.scores = ptr(scores)
    args.gates = ptr(gates)
    args.workspace = ptr(ws)
    args.workspace_bytes = ws.numel()
    args.tokens, args.hidden_size, args.expert_count, args.top_k = tokens, hidden, experts, top_k
    args.act_dtype = act_code(x)
    args.renorm_blend = float(renorm_blend)
    _lib.check(lib.vm_router_topk(args, stream_handle()))
    if return_gates:
        return inds, scores, gates
    return inds, scores
