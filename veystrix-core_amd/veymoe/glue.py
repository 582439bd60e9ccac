"""Decoder glue around the MoE call: the hyper-connection of the MLP branch.

In the reference's decoder layer the MoE branch sits between two pieces of
glue (compile_glue.py:44-61, ``_decoder_call``):

    mixed, hyper_input, weights = self.mlp_hyper_connection(hidden)
    branch = self.mlp(mixed)                       # the MoE layer
    hidden = _inject(hyper_input, branch, weights) # compile_glue.py:32-35

The hyper-connection (qwen4_verifier.py:20-33, ``_hyper``) normalises the
``hc`` residual streams with ``hc_norm`` (an RMSNorm, patch_rmsnorm.py:108-135),
mixes them into the branch input through two low-rank Q4/G32 projections and
derives one injection weight per stream.  Here:

* ``HyperConnection(hidden)`` runs it as ``vm_hyper_mix`` (two launches);
* ``mlp_branch(hyper, moe, hidden)`` runs the whole branch: the
  hyper-connection, then the MoE layer with the injection written by the
  experts' final epilogue (no launch of its own).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .device import act_code, ptr, q4proj, require_device, stream_handle
from .executor import Q4G32Projection
from .layer import MoELayer


def _rows(proj: Q4G32Projection):
    shape = tuple(proj.weight.shape)
    return shape[-2], shape[-1] * 8     # (out, in)


class HyperConnection:
    """``Qwen4ExpGatedResidual`` of one branch: hc_norm gain [hc*H],
    ``input_mix_weight_down`` [lowrank, hc*H], ``input_mix_weight_up``
    [hc*H, lowrank] and ``block_inject_weight`` [hc, hc*H], Q4/G32.
    ``norm_group`` 0 normalises the whole row (else groups of that size);
    ``one_centered`` chooses the gain convention (patch_rmsnorm.py:62-66)."""

    def __init__(self, norm_weight: torch.Tensor, mix_down: Q4G32Projection, mix_up: Q4G32Projection,
                 inject: Q4G32Projection, hc_count: int, *, eps: float = 1e-6, norm_group: int = 0,
                 one_centered: bool = True):
        hc = int(hc_count)
        n = norm_weight.numel()
        if hc < 1 or hc > _lib.VM_MAX_STREAMS or n % hc:
            raise ValueError(f"hc_count must be 1..{_lib.VM_MAX_STREAMS} and divide the row")
        lowrank, down_in = _rows(mix_down)
        up_out, up_in = _rows(mix_up)
        inj_out, inj_in = _rows(inject)
        if down_in != n or up_out != n or up_in != lowrank or inj_out != hc or inj_in != n:
            raise ValueError("projection shapes must be [lowrank, n], [n, lowrank] and [hc, n]")
        self.norm_weight = norm_weight.reshape(-1).contiguous()
        self.mix_down, self.mix_up, self.inject = mix_down, mix_up, inject
        self.hc_count = hc
        self.hidden_size = n // hc
        self.lowrank = lowrank
        self.eps = float(eps)
        self.norm_group = int(norm_group)
        self.one_centered = bool(one_centered)
        self._gain = {}
        self._ws = {}

    def _gain_of(self, dtype):
        g = self._gain.get(dtype)
        if g is None:
            g = self.norm_weight.to(dtype).contiguous()
            self._gain[dtype] = g
        return g

    def __call__(self, hidden: torch.Tensor):
        """(mixed [..., H], hidden, weights [..., hc]) of hidden [..., hc*H]."""
        n = self.hc_count * self.hidden_size
        if hidden.shape[-1] != n:
            raise ValueError(f"hidden must end in {n} values")
        flat = hidden.reshape(-1, n).contiguous()
        require_device("hidden", flat, (torch.bfloat16, torch.float32))
        T = flat.shape[0]
        lib = _lib.lib()
        dtype = act_code(flat)
        key = (T, dtype, flat.device)
        ws = self._ws.get(key)
        if ws is None:
            nbytes = int(lib.vm_hyper_mix_workspace(T, self.hc_count, self.hidden_size, self.lowrank, dtype))
            ws = torch.empty(nbytes, dtype=torch.uint8, device=flat.device)
            self._ws[key] = ws
        mixed = torch.empty((T, self.hidden_size), dtype=flat.dtype, device=flat.device)
        weights = torch.empty((T, self.hc_count), dtype=flat.dtype, device=flat.device)
        a = _lib.VmHyperArgs()
        a.hidden = ptr(flat)
        a.norm_weight = ptr(self._gain_of(flat.dtype))
        a.mix_down = q4proj(self.mix_down.weight, self.mix_down.scales, self.mix_down.biases)
        a.mix_up = q4proj(self.mix_up.weight, self.mix_up.scales, self.mix_up.biases)
        a.inject = q4proj(self.inject.weight, self.inject.scales, self.inject.biases)
        a.mixed = ptr(mixed)
        a.weights = ptr(weights)
        a.workspace = ptr(ws)
        a.workspace_bytes = ws.numel()
        a.tokens, a.hidden_size, a.hc_count, a.lowrank = T, self.hidden_size, self.hc_count, self.lowrank
        a.norm_group, a.one_centered = self.norm_group, int(self.one_centered)
        a.act_dtype = dtype
        a.eps = self.eps
        _lib.check(lib.vm_hyper_mix(ctypes.byref(a), stream_handle()))
        lead = hidden.shape[:-1]
        return mixed.reshape(*lead, self.hidden_size), hidden, weights.reshape(*lead, self.hc_count)


def mlp_branch(hyper: HyperConnection, moe: MoELayer, hidden: torch.Tensor, out: torch.Tensor = None):
    """The decoder layer's MLP branch on hidden [..., hc*H]: hyper-connection,
    MoE layer, injection (compile_glue.py:58-61).  Returns the new hidden
    state (``out``, which may be ``hidden`` itself, or a new tensor)."""
    if moe.hidden != hyper.hidden_size:
        raise ValueError("the MoE layer's hidden size must be the hyper-connection's")
    n = hyper.hc_count * hyper.hidden_size
    streams = hidden.reshape(-1, n)
    if not streams.is_contiguous():
        streams = streams.contiguous()
    mixed, _, weights = hyper(streams)
    target = torch.empty_like(streams) if out is None else out.reshape(-1, n)
    moe.forward(mixed, inject=(streams, weights, target))
    return target.reshape(hidden.shape)


__all__ = ["HyperConnection", "mlp_branch"]
