"""Brute-force pure-Python loops for tiny shapes.

TEST INFRASTRUCTURE ONLY (see oracle/moe_oracle.py).

``projection_loops`` is a line-by-line restatement of the loop nest of the
reference's ``_numpy_projection`` (models/flashnext/metal_runtime.py:997-1029):
per (token, slot, row) a Python-float accumulation over groups, each group
summing ``value*q`` and ``value`` over its 32 inputs, then
``result += scale*qsum; result += bias*xsum``.  It exists to pin the vectorised
``moe_oracle.q4_project`` on tiny shapes, with an independent nibble decode
(plain integer shifts on Python ints).

``qmm_loops`` restates the matrix form used for more than 8 rows (weights
dequantised and rounded to bf16 before the multiply) with its own bf16
rounding on the float32 bit pattern, to pin ``moe_oracle.qmm_project``.
"""
from __future__ import annotations

import struct


def _bf16_value(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", (int(bits) & 0xFFFF) << 16))[0]


def projection_loops(x, routes, weight, scales, biases, output_width, slot_input,
                     group_size=32):
    """x: nested lists [tokens][in] (or [tokens][slots][in] when slot_input);
    routes: [tokens][slots] ints; weight: [E][out][in/8] ints;
    scales/biases: [E][out][in/group] bf16 bit patterns.
    Returns nested lists [tokens][slots][out] of Python floats."""
    tokens = len(routes)
    slots = len(routes[0])
    out = []
    for token in range(tokens):
        token_out = []
        for slot in range(slots):
            expert = int(routes[token][slot])
            source = x[token][slot] if slot_input else x[token]
            input_width = len(source)
            rows = []
            for row in range(output_width):
                result = 0.0
                for group in range(input_width // group_size):
                    qsum = 0.0
                    xsum = 0.0
                    for i in range(group_size):
                        k = group * group_size + i
                        q = (int(weight[expert][row][k // 8]) >> ((k & 7) * 4)) & 15
                        value = float(source[k])
                        qsum += value * q
                        xsum += value
                    result += _bf16_value(scales[expert][row][group]) * qsum
                    result += _bf16_value(biases[expert][row][group]) * xsum
                rows.append(result)
            token_out.append(rows)
        out.append(token_out)
    return out


def _round_bf16_value(value: float) -> float:
    """float32(value) rounded to bf16, nearest-even, by integer arithmetic on
    the float32 bit pattern (an independent restatement of the rounding)."""
    bits = struct.unpack("<I", struct.pack("<f", value))[0]
    if (bits & 0x7F800000) == 0x7F800000:
        return struct.unpack("<f", struct.pack("<I", bits & 0xFFFF0000))[0]
    lower = bits & 0xFFFF
    upper = bits >> 16
    if lower > 0x8000 or (lower == 0x8000 and (upper & 1)):
        upper += 1
    return struct.unpack("<f", struct.pack("<I", (upper & 0xFFFF) << 16))[0]


def qmm_loops(x, weight, scales, biases, group_size=32):
    """Matrix form for one expert on rows x [n][in]: every weight dequantised
    as float32(scale*q + bias) rounded to bf16, then plain dot products.
    weight: [out][in/8] ints; scales/biases [out][in/group] bf16 bits."""
    out = []
    for row_x in x:
        row_out = []
        for row in range(len(weight)):
            acc = 0.0
            for k in range(len(row_x)):
                q = (int(weight[row][k // 8]) >> ((k & 7) * 4)) & 15
                group = k // group_size
                w = _bf16_value(scales[row][group]) * q + _bf16_value(biases[row][group])
                acc += float(row_x[k]) * _round_bf16_value(w)
            row_out.append(acc)
        out.append(row_out)
    return out


def pack_nibbles(values):
    """Inverse of the MLX nibble order for one row: ints 0..15 -> uint32 words."""
    if len(values) % 8:
        raise ValueError("row length must be a multiple of 8")
    words = []
    for w in range(len(values) // 8):
        word = 0
        for n in range(8):
            q = int(values[8 * w + n])
            if not 0 <= q <= 15:
                raise ValueError("nibble out of range")
            word |= q << (4 * n)
        words.append(word)
    return words
