"""Torch plumbing for the C ABI: device pointers, dtype codes, streams."""
from __future__ import annotations

import ctypes

import torch

from . import _lib

ACT_DTYPES = {torch.bfloat16: _lib.VM_BF16, torch.float32: _lib.VM_F32}
_WORD_DTYPES = (torch.int32, getattr(torch, "uint32", torch.int32))


def shape_of(value):
    return tuple(int(v) for v in value.shape)


def require_device(name: str, tensor, dtypes=None):
    """Check that ``tensor`` is a contiguous tensor on the GPU (optionally of a dtype)."""
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor on the GPU, got {type(tensor).__name__}")
    if tensor.device.type != "cuda":
        raise TypeError(f"{name} must live on the GPU (got {tensor.device})")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtypes is not None and tensor.dtype not in dtypes:
        raise TypeError(f"{name} has dtype {tensor.dtype}; expected one of {dtypes}")
    return tensor


def ptr(tensor) -> int | None:
    if tensor is None:
        return None
    return tensor.data_ptr()


def act_code(tensor) -> int:
    try:
        return ACT_DTYPES[tensor.dtype]
    except KeyError:
        raise TypeError(f"activations must be bfloat16 or float32, got {tensor.dtype}") from None


def word_tensor(name: str, tensor):
    """Route words / packed weights: int32 or uint32 tensors on the GPU."""
    require_device(name, tensor)
    if tensor.dtype not in _WORD_DTYPES:
        raise TypeError(f"{name} must use 32-bit packed values (int32/uint32), got {tensor.dtype}")
    return tensor


def stream_handle(stream=None) -> ctypes.c_void_p:
    stream = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(stream.cuda_stream)


def q4proj(weight=None, scales=None, biases=None) -> _lib.VmQ4Proj:
    return _lib.VmQ4Proj(ptr(weight), ptr(scales), ptr(biases))


def workspace(nbytes: int, device) -> torch.Tensor:
    """Zero-initialised device scratch (counters in it must start at zero)."""
    return torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)
