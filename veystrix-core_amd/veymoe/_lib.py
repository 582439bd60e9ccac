"""ctypes binding of libveymoe.so (the C ABI declared in include/veymoe.h).

The library is built in-tree by ``veymoe.build.build()``.  There is no
fallback: when the shared object is missing or the device is not a gfx950,
every compute entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libveymoe.so")

VM_OK = 0
VM_EINVAL = -1
VM_EUNSUPPORTED = -2
VM_EHIP = -3
VM_EWORKSPACE = -4
VM_STATIC_SCRATCH_BYTES = 4 << 20  # vm_moe_layer_static's per-device scratch
VM_BF16 = 0
VM_F32 = 1
VM_SLOT_BIT = 0x80000000
VM_PARTS = 9

_c_u32 = ctypes.c_uint32
_c_u64 = ctypes.c_uint64
_vp = ctypes.c_void_p


class VmQ4Proj(ctypes.Structure):
    _fields_ = [("weight", _vp), ("scales", _vp), ("biases", _vp)]


class VmPoolView(ctypes.Structure):
    _fields_ = [
        ("base", _vp),
        ("header_size", _c_u64),
        ("record_stride", _c_u64),
        ("part_offset", _c_u64 * VM_PARTS),
        ("records", _c_u32),
        ("reserved", _c_u32),
    ]


class VmMoeArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp),
        ("gate", VmQ4Proj), ("up", VmQ4Proj), ("down", VmQ4Proj),
        ("pool", VmPoolView),
        ("stream", VmPoolView),
        ("routes", _vp),
        ("slot_table", _vp),
        ("scores", _vp),
        ("shared_y", _vp),
        ("shared", _vp),
        ("shared_gate", _vp),
        ("activation_in", _vp),
        ("activation_out", _vp),
        ("gate_out", _vp),
        ("up_out", _vp),
        ("output", _vp),
        ("status", _vp),
        ("workspace", _vp),
        ("workspace_bytes", _c_u64),
        ("tokens", _c_u32), ("slots", _c_u32), ("hidden_size", _c_u32), ("inter_size", _c_u32),
        ("expert_count", _c_u32), ("group_size", _c_u32),
        ("act_dtype", _c_u32), ("score_dtype", _c_u32),
    ]


class VmRouterArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp),
        ("weight", _vp),
        ("logit_bias", _vp),
        ("inds", _vp),
        ("scores", _vp),
        ("gates", _vp),
        ("workspace", _vp),
        ("workspace_bytes", _c_u64),
        ("tokens", _c_u32), ("hidden_size", _c_u32), ("expert_count", _c_u32), ("top_k", _c_u32),
        ("act_dtype", _c_u32),
        ("renorm_blend", ctypes.c_float),
    ]


class VmLayerArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp),
        ("output", _vp),
        ("router_weight", _vp),
        ("router_bias", _vp),
        ("gate", VmQ4Proj), ("up", VmQ4Proj), ("down", VmQ4Proj),
        ("pool", VmPoolView),
        ("slot_table", _vp),
        ("shared_gate_proj", VmQ4Proj), ("shared_up_proj", VmQ4Proj), ("shared_down_proj", VmQ4Proj),
        ("shared_expert_gate", VmQ4Proj),
        ("inds_out", _vp),
        ("scores_out", _vp),
        ("status", _vp),
        ("workspace", _vp),
        ("workspace_bytes", _c_u64),
        ("tokens", _c_u32), ("hidden_size", _c_u32), ("inter_size", _c_u32), ("shared_inter", _c_u32),
        ("expert_count", _c_u32), ("top_k", _c_u32), ("group_size", _c_u32),
        ("act_dtype", _c_u32),
        ("renorm_blend", ctypes.c_float),
        ("phases", _c_u32),
        ("inject_hidden", _vp),
        ("inject_weights", _vp),
        ("inject_out", _vp),
        ("hc_count", _c_u32),
        ("combine", _c_u32),
        ("gates_out", _vp),
    ]


VM_COMBINE_FUSED = 0
VM_COMBINE_GENERIC = 1
VM_PHASE_ROUTER = 1
VM_PHASE_EXPERTS = 2
VM_MAX_STREAMS = 8


class VmHyperArgs(ctypes.Structure):
    _fields_ = [
        ("hidden", _vp),
        ("norm_weight", _vp),
        ("mix_down", VmQ4Proj), ("mix_up", VmQ4Proj), ("inject", VmQ4Proj),
        ("mixed", _vp),
        ("weights", _vp),
        ("normed", _vp),
        ("workspace", _vp),
        ("workspace_bytes", _c_u64),
        ("tokens", _c_u32), ("hidden_size", _c_u32), ("hc_count", _c_u32), ("lowrank", _c_u32),
        ("norm_group", _c_u32), ("one_centered", _c_u32),
        ("act_dtype", _c_u32),
        ("eps", ctypes.c_float),
    ]


class VmDeviceLru(ctypes.Structure):
    _fields_ = [
        ("slot_table", _vp),
        ("slot_owner", _vp),
        ("lru_order", _vp),
        ("counters", _vp),
        ("host_row", _vp),
        ("host_store", _vp),
        ("host_stride", _c_u64),
        ("host_records", _c_u64),
        ("layers", _c_u32),
        ("layer", _c_u32),
        ("slots", _c_u32),
        ("order_len", _c_u32),
    ]


class VmGroupedArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp),
        ("inds", _vp),
        ("scores", _vp),
        ("gate", VmQ4Proj), ("up", VmQ4Proj), ("down", VmQ4Proj),
        ("pool", VmPoolView),
        ("slot_table", _vp),
        ("shared_y", _vp),
        ("output", _vp),
        ("status", _vp),
        ("workspace", _vp),
        ("workspace_bytes", _c_u64),
        ("tokens", _c_u32), ("top_k", _c_u32), ("hidden_size", _c_u32), ("inter_size", _c_u32),
        ("expert_count", _c_u32), ("group_size", _c_u32),
        ("act_dtype", _c_u32), ("combine_mode", _c_u32),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "vm_abi_version": (ctypes.c_int, []),
    "vm_available": (ctypes.c_int, []),
    "vm_last_error": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t]),
    "vm_moe_execute_workspace": (_c_u64, [_c_u32, _c_u32, _c_u32, _c_u32]),
    "vm_moe_execute": (ctypes.c_int, [ctypes.POINTER(VmMoeArgs), _vp]),
    "vm_router_workspace": (_c_u64, [_c_u32, _c_u32]),
    "vm_router_topk": (ctypes.c_int, [ctypes.POINTER(VmRouterArgs), _vp]),
    "vm_moe_layer_workspace": (_c_u64, [_c_u32, _c_u32, _c_u32, _c_u32, _c_u32, _c_u32, _c_u32]),
    "vm_moe_layer": (ctypes.c_int, [ctypes.POINTER(VmLayerArgs), _vp]),
    "vm_moe_layer_lru": (ctypes.c_int, [ctypes.POINTER(VmLayerArgs), ctypes.POINTER(VmDeviceLru), _vp]),
    "vm_moe_layer_static": (ctypes.c_int, [ctypes.POINTER(VmLayerArgs), _vp]),
    "vm_hyper_mix_workspace": (_c_u64, [_c_u32, _c_u32, _c_u32, _c_u32, _c_u32]),
    "vm_hyper_mix": (ctypes.c_int, [ctypes.POINTER(VmHyperArgs), _vp]),
    "vm_moe_grouped_workspace": (_c_u64, [_c_u32, _c_u32, _c_u32, _c_u32, _c_u32, _c_u32]),
    "vm_moe_grouped": (ctypes.c_int, [ctypes.POINTER(VmGroupedArgs), _vp]),
    "vm_weighted_combine": (ctypes.c_int, [_vp, _vp, _vp, _c_u32, _c_u32, _c_u32, _c_u32, _c_u32, _vp]),
    "vm_pool_stage": (ctypes.c_int, [_vp, _c_u64, _c_u64, _c_u64, _vp, _c_u64, _c_u64, _c_u64,
                                     ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64),
                                     _c_u32, _vp]),
    "vm_decode_pipeline": (ctypes.c_int, [ctypes.c_int]),
    "vm_timing_enable": (ctypes.c_int, [ctypes.c_int]),
    "vm_timing_read": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_uint64)]),
    "vm_timing_reset": (ctypes.c_int, []),
    "vm_trace_set": (ctypes.c_int, [_vp, _c_u64]),
    "vm_trace_records": (_c_u64, []),
}


class ExtensionMissing(RuntimeError):
    """libveymoe.so is not built; run ``python -c 'import __graft_entry__ as g; g.build()'``."""


class VeymoeError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"libveymoe error {code}: {message}")
        self.code = code


_LOCK = threading.Lock()
_LIB = None


def lib():
    """The loaded library (ctypes.CDLL) with argument types set."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not os.path.exists(LIB_PATH):
                raise ExtensionMissing(
                    f"{LIB_PATH} is missing: the HIP extension has not been built "
                    "(python -c 'import __graft_entry__ as g; g.build()')")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _LIB = handle
    return _LIB


def last_error() -> str:
    buf = ctypes.create_string_buffer(512)
    lib().vm_last_error(buf, len(buf))
    return buf.value.decode("utf-8", "replace")


def check(code: int) -> None:
    if code != VM_OK:
        message = last_error()
        if code == VM_EINVAL:
            raise ValueError(message)
        raise VeymoeError(code, message)


def lib_built_with_fused_pipelines():
    """Whether the built library carries the one-token pipelines 1 and 2 (a
    library built with -DVM_FUSED_PIPELINES=1); None when it is not built."""
    if not os.path.exists(LIB_PATH):
        return None
    handle = lib()
    previous = handle.vm_decode_pipeline(-1)
    rc = handle.vm_decode_pipeline(1)
    if rc < 0:
        return False
    handle.vm_decode_pipeline(previous)
    return True
