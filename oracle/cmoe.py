"""ctypes wrapper of oracle/libcmoe.so (the C restatement, CPU baseline).

TEST INFRASTRUCTURE ONLY (see oracle/moe_oracle.py).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from .build import LIB


class CmoeQ4(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("b", ctypes.c_void_p)]


class CmoeLayer(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int), ("inter", ctypes.c_int), ("experts", ctypes.c_int), ("top_k", ctypes.c_int),
        ("shared_inter", ctypes.c_int),
        ("router", ctypes.c_void_p), ("router_bias", ctypes.c_void_p),
        ("records", ctypes.c_void_p), ("record_stride", ctypes.c_uint64), ("offsets", ctypes.c_uint64 * 9),
        ("record_of", ctypes.c_void_p),
        ("sgate", CmoeQ4), ("sup", CmoeQ4), ("sdown", CmoeQ4), ("segate", CmoeQ4),
    ]


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built (oracle.build.build())")
        _LIB = ctypes.CDLL(LIB)
        _LIB.cmoe_decode_token.restype = ctypes.c_int
        _LIB.cmoe_decode_token.argtypes = [ctypes.POINTER(CmoeLayer), ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        _LIB.cmoe_scratch_floats.restype = ctypes.c_int
        _LIB.cmoe_scratch_floats.argtypes = [ctypes.c_int] * 4
        _LIB.cmoe_threads.restype = ctypes.c_int
    return _LIB


def _p(a):
    return None if a is None else a.ctypes.data


class CDecodeLayer:
    """Holds the arrays of one layer and runs decode tokens through the C code."""

    def __init__(self, hidden, inter, experts, top_k, router_bits, records, record_stride, offsets,
                 router_bias=None, record_of=None, shared=None):
        self._keep = []

        def keep(a, dtype):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=dtype)
            self._keep.append(a)
            return a

        self.layer = CmoeLayer()
        L = self.layer
        L.hidden, L.inter, L.experts, L.top_k = hidden, inter, experts, top_k
        L.router = _p(keep(router_bits, np.uint16))
        L.router_bias = _p(keep(router_bias, np.float32))
        L.records = _p(keep(records, np.uint8))
        L.record_stride = record_stride
        for i, off in enumerate(offsets):
            L.offsets[i] = off
        L.record_of = _p(keep(record_of, np.int32))
        if shared is not None:
            L.shared_inter = int(np.asarray(shared["gate_proj"][0]).shape[-2])
            for field, key in (("sgate", "gate_proj"), ("sup", "up_proj"), ("sdown", "down_proj"),
                               ("segate", "gate")):
                w, s, b = shared[key]
                setattr(L, field, CmoeQ4(_p(keep(w, np.uint32)), _p(keep(s, np.uint16)), _p(keep(b, np.uint16))))
        self.top_k = top_k
        self.hidden = hidden
        self.scratch = np.zeros(lib().cmoe_scratch_floats(hidden, inter, experts, top_k), dtype=np.float32)

    def run(self, x_bits):
        """x_bits [H] uint16 -> (inds [k] int32, scores [k] float32, y bits [H] uint16)."""
        x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
        inds = np.zeros(self.top_k, dtype=np.int32)
        scores = np.zeros(self.top_k, dtype=np.float32)
        y = np.zeros(self.hidden, dtype=np.uint16)
        lib().cmoe_decode_token(ctypes.byref(self.layer), _p(x_bits), _p(inds), _p(scores), _p(y),
                                _p(self.scratch))
        return inds, scores, y


def threads() -> int:
    return int(lib().cmoe_threads())
