"""Expert record layout and packing.

An expert record holds the nine quantized parts of one expert back to back,
in the order of the reference's slab record (models/flashnext/slab_pack.py:96-149,
expert_pool.py:45-49):

    gate_proj.{weight, scales, biases}, up_proj.{...}, down_proj.{...}

weight parts are uint32 ``[out, in/8]``, scales/biases bf16 ``[out, in/32]``.
The reference hard-codes hidden 2560 / intermediate 640 (3,072,000-byte
records); here the sizes are parameters, and the stride is rounded up to a
4 KiB page (the reference asserts page alignment instead; both agree wherever
the reference's layout exists).  A pool or pack region starts with a
``header_size`` (4 KiB) header, then record r at ``header + r * stride``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Tuple

import numpy as np

PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
PART_NAMES = ("weight", "scales", "biases")
PARTS = tuple((proj, part) for proj in PROJECTIONS for part in PART_NAMES)
HEADER = 4096
PAGE = 4096
SLOT_BIT = 0x80000000


@dataclass(frozen=True)
class RecordLayout:
    hidden: int
    inter: int
    group_size: int = 32
    page: int = PAGE
    offsets: Dict[Tuple[str, str], int] = field(init=False, compare=False)
    sizes: Dict[Tuple[str, str], int] = field(init=False, compare=False)
    record_stride: int = field(init=False, compare=False)
    record_bytes: int = field(init=False, compare=False)

    def __post_init__(self):
        if self.hidden % self.group_size or self.inter % self.group_size:
            raise ValueError("hidden and intermediate sizes must be multiples of the group size")
        offsets, sizes = {}, {}
        cursor = 0
        for proj, part in PARTS:
            rows, cols = self.shape(proj, part)
            size = rows * cols * (4 if part == "weight" else 2)
            offsets[(proj, part)] = cursor
            sizes[(proj, part)] = size
            cursor += size
        object.__setattr__(self, "offsets", offsets)
        object.__setattr__(self, "sizes", sizes)
        object.__setattr__(self, "record_bytes", cursor)
        object.__setattr__(self, "record_stride", -(-cursor // self.page) * self.page)

    def in_out(self, proj: str) -> Tuple[int, int]:
        """(input width, output width) of a projection."""
        if proj == "down_proj":
            return self.inter, self.hidden
        return self.hidden, self.inter

    def shape(self, proj: str, part: str) -> Tuple[int, int]:
        """Element shape of one part: weight (out, in/8) uint32, else (out, in/group)."""
        in_width, out_width = self.in_out(proj)
        if part == "weight":
            return out_width, in_width // 8
        return out_width, in_width // self.group_size

    def offset(self, proj: str, part: str) -> int:
        return self.offsets[(proj, part)]

    def part_offsets(self):
        return [self.offsets[key] for key in PARTS]

    @property
    def expert_bytes(self) -> int:
        """Algorithmic bytes of one expert (all nine parts): 1.875 * I * H for G32."""
        return self.record_bytes


def pack_record(parts: Dict[Tuple[str, str], np.ndarray], layout: RecordLayout,
                out: np.ndarray | None = None) -> np.ndarray:
    """Pack one expert's nine parts (numpy; weights uint32, metadata uint16 bf16
    bits) into a uint8 record of ``layout.record_stride`` bytes."""
    if out is None:
        out = np.zeros(layout.record_stride, dtype=np.uint8)
    for key in PARTS:
        value = np.ascontiguousarray(parts[key])
        expected_dtype = np.uint32 if key[1] == "weight" else np.uint16
        if value.dtype != expected_dtype or value.shape != layout.shape(*key):
            raise ValueError(f"{key[0]}.{key[1]} must be {expected_dtype.__name__} {layout.shape(*key)}, "
                             f"got {value.dtype} {value.shape}")
        start = layout.offset(*key)
        raw = value.view(np.uint8).reshape(-1)
        out[start:start + raw.size] = raw
    return out


def unpack_record(record: np.ndarray, layout: RecordLayout) -> Dict[Tuple[str, str], np.ndarray]:
    """Inverse of pack_record (views into ``record``)."""
    parts = {}
    for key in PARTS:
        start = layout.offset(*key)
        dtype = np.uint32 if key[1] == "weight" else np.uint16
        size = layout.sizes[key]
        parts[key] = record[start:start + size].view(dtype).reshape(layout.shape(*key))
    return parts
