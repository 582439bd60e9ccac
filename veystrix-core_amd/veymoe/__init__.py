"""veymoe: the routed-expert MoE layer of Veystrix Flash-Next on MI355X (gfx950).

Host code in Python on PyTorch-ROCm (device memory and streams); compute in
hand-written HIP kernels behind the C ABI of ``include/veymoe.h``
(``libveymoe.so``, loaded with ctypes).

Public surface (reference counterparts in joyboyreturns/Veystrix-Core):
  HipMoEExecutor / weighted_combine / probe_capabilities   metal_runtime.py
  MoELayer (the _moe_call block), HipSwitchGLU              adaptive_topk.py, expert_cache.py
  ExpertPool / HostRecordStore                              expert_pool.py
  RecordLayout                                              slab_pack.py
  router_topk                                               compiled.py
"""
from .executor import (BITS, GROUP_SIZE, MAX_EXPERTS, MAX_TOKENS, MAX_TOP_K, MAX_WIDTH, HipCapabilities,
                       HipMoEExecutor, Q4G32Projection, probe_capabilities, weighted_combine)
from .layout import HEADER, PARTS, SLOT_BIT, RecordLayout, pack_record, unpack_record

__all__ = [
    "BITS", "GROUP_SIZE", "HEADER", "MAX_EXPERTS", "MAX_TOKENS", "MAX_TOP_K", "MAX_WIDTH", "PARTS", "SLOT_BIT",
    "HipCapabilities", "HipMoEExecutor", "Q4G32Projection", "RecordLayout", "pack_record", "probe_capabilities",
    "unpack_record", "weighted_combine",
]
