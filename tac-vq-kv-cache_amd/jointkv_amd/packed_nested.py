"""LSB-first fixed-width index packing (host byte streams).

Same byte format as src/jointkv/packed_nested.py:30-72: value i occupies
bits [i*w, (i+1)*w) of the stream, least-significant bit first, and the last
byte is zero-padded.  For 8-bit codes the stream equals the code bytes.
Implemented with numpy bit operations on host memory.
"""

from __future__ import annotations

import numpy as np
import torch


def pack_fixed_width(values: torch.Tensor, bits: int) -> torch.Tensor:
    """Pack non-negative integers < 2**bits into an LSB-first uint8 stream."""

    width = int(bits)
    if width <= 0 or width > 8:
        raise ValueError("bits must lie in [1, 8]")
    flat = values.detach().to(device="cpu", dtype=torch.int64).reshape(-1).numpy()
    if flat.size == 0:
        return torch.empty(0, dtype=torch.uint8)
    if (flat < 0).any() or (flat >= (1 << width)).any():
        raise ValueError(f"a value is outside the unsigned {width}-bit range")
    bit_matrix = ((flat[:, None] >> np.arange(width)) & 1).astype(np.uint8)
    packed = np.packbits(bit_matrix.reshape(-1), bitorder="little")
    return torch.from_numpy(packed.copy())


def unpack_fixed_width(packed: torch.Tensor, bits: int, count: int) -> torch.Tensor:
    """Invert :func:`pack_fixed_width`; returns ``count`` uint8 values."""

    width = int(bits)
    number = int(count)
    if width <= 0 or width > 8:
        raise ValueError("bits must lie in [1, 8]")
    if number < 0:
        raise ValueError("count must be non-negative")
    expected = (number * width + 7) // 8
    stream = packed.detach().to(device="cpu", dtype=torch.uint8).reshape(-1).numpy()
    if stream.size != expected:
        raise ValueError(f"packed stream has {stream.size} bytes, expected {expected}")
    if number == 0:
        return torch.empty(0, dtype=torch.uint8)
    bit_stream = np.unpackbits(stream, bitorder="little")[: number * width]
    weights = (1 << np.arange(width)).astype(np.uint16)
    values = (bit_stream.reshape(number, width).astype(np.uint16) * weights).sum(axis=1)
    return torch.from_numpy(values.astype(np.uint8))
