"""The grouped expert block (rows > 8): SwitchGLU over expert ids on the
device token-by-expert sort and the MFMA grouped kernels (vm_moe_grouped).

Mirrors the reference's generic ``gather_qmm`` path of
``StreamingSwitchGLU._one_pass`` (models/flashnext/expert_cache.py:1949-2037):
per-slot expert outputs ``[rows, k, hidden]`` (combine mode 2), or the
combined ``[rows, hidden]`` with the generic (1) or fused (0) combine.
"""
from __future__ import annotations

import torch

from . import _lib
from .device import ptr, q4proj, require_device, stream_handle

COMBINE_FUSED, COMBINE_GENERIC, COMBINE_NONE = 0, 1, 2


def grouped_experts(switch, x: torch.Tensor, inds: torch.Tensor, scores: torch.Tensor = None,
                    shared_y: torch.Tensor = None, mode: int = COMBINE_NONE) -> torch.Tensor:
    """x [rows, hidden] bf16, inds [rows, k] expert ids -> [rows, k, hidden]
    (mode 2) or [rows, hidden] (modes 0/1, scores required)."""
    require_device("x", x, (torch.bfloat16,))
    rows, k = inds.shape
    inds = inds.to(torch.int32).contiguous()
    lib = _lib.lib()
    a = _lib.VmGroupedArgs()
    a.x = ptr(x)
    a.inds = ptr(inds)
    if mode != COMBINE_NONE:
        if scores is None:
            raise ValueError("scores are required to combine")
        scores = require_device("scores", scores.reshape(rows, k).to(torch.bfloat16).contiguous())
        a.scores = ptr(scores)
        out = torch.empty((rows, switch.hidden), dtype=x.dtype, device=x.device)
    else:
        out = torch.empty((rows, k, switch.hidden), dtype=x.dtype, device=x.device)
    if shared_y is not None:
        shared_y = require_device("shared_y", shared_y.reshape(rows, switch.hidden).to(x.dtype).contiguous())
        a.shared_y = ptr(shared_y)
    if switch.pool is not None:
        pool = switch.pool
        routed = inds.reshape(-1).tolist()  # route sync for the host LRU pass
        wanted = list(dict.fromkeys(routed))
        _, misses = pool.assign(switch.layer_id, wanted)
        switch.hits += len(routed) - len(misses)
        switch.misses += len(misses)
        if misses:
            if switch.host_store is None:
                pool.invalidate(switch.layer_id, misses)
                raise RuntimeError("expert pool miss with no host record store to fill from")
            pool.fill(switch.layer_id, misses, switch.host_store)
        pool.sync_tables()
        a.pool = pool.view()
        a.slot_table = ptr(pool.table(switch.layer_id))
    else:
        a.gate = q4proj(switch.gate_proj.weight, switch.gate_proj.scales, switch.gate_proj.biases)
        a.up = q4proj(switch.up_proj.weight, switch.up_proj.scales, switch.up_proj.biases)
        a.down = q4proj(switch.down_proj.weight, switch.down_proj.scales, switch.down_proj.biases)
    nbytes = int(lib.vm_moe_grouped_workspace(rows, k, switch.hidden, switch.inter, switch.num_experts, 0))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    a.output = ptr(out)
    a.workspace = ptr(ws)
    a.workspace_bytes = nbytes
    a.tokens, a.top_k = rows, k
    a.hidden_size, a.inter_size, a.expert_count = switch.hidden, switch.inter, switch.num_experts
    a.group_size = switch.group_size
    a.act_dtype = 0
    a.combine_mode = mode
    _lib.check(lib.vm_moe_grouped(a, stream_handle()))
    return out


__all__ = ["COMBINE_FUSED", "COMBINE_GENERIC", "COMBINE_NONE", "grouped_experts"]
