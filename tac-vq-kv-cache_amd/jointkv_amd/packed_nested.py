"""Bit-packed code streams on the host: fixed-width packing and the paired
progressive K/V layout with its byte ledger.

Same byte formats and ledgers as src/jointkv/packed_nested.py:

* ``pack_fixed_width`` (:30-72): value i occupies bits [i*w, (i+1)*w) of the
  stream, least-significant bit first; the last byte is zero-padded.  For
  8-bit codes the stream equals the code bytes.
* The progressive layout (:547-601 pack, :604-681 unpack, :684-734
  validation).  A unit (batch, head, token) has one of three depths
  ``exits = (e0, e1, e2)``; its stage indices are split into tiers
      base  stages [0, e0)   every unit,
      mid   stages [e0, e1)  units with depth >= e1,
      high  stages [e1, e2)  units with depth == e2,
  and tokens are cut into blocks of ``block_size`` along each (batch, head)
  row.  A tier's stream is, block after block (row-major), one byte-aligned
  segment per stage of the tier holding the block's selected tokens in token
  order at that stage's width.  mid/high carry int32 block offsets; base
  offsets follow from the geometry.  A shared 2-bit label per unit names its
  exit (code 3 is reserved).
* Ledgers: ``estimate_paired_progressive_layout`` (:210-309, exact bytes of
  the layout above without packing), its per-layer sum (:312-365) and the
  block-shared variant (:368-451, one depth per token block, one stream per
  stage, no offsets).

The reference loops over blocks and stages; here every tier is laid out in
one pass: per-block counts give each (block, stage) segment its byte start,
each selected token its bit address (start * 8 + rank-in-block * width), and
the bits land by vectorised numpy scatter, so packing costs O(total bits).
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Sequence

import numpy as np
import torch

from .budget import prefix_index_bits, validate_stage_bits

_INT32_MAX = int(np.iinfo(np.int32).max)


def _ceil_div(a, b):
    return (a + b - 1) // b


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


# ---------------------------------------------------------------------------
# Containers and ledger


@dataclass(frozen=True)
class PackedProgressiveStream:
    """The base, mid and high byte streams of one kind (K or V)."""

    base: torch.Tensor
    mid: torch.Tensor
    high: torch.Tensor

    @property
    def allocated_bytes(self) -> int:
        return sum(int(t.numel() * t.element_size()) for t in (self.base, self.mid, self.high))


@dataclass(frozen=True)
class PackedLayoutLedger:
    """Physical bit inventory of one packed K/V layout."""

    payload_bits: int
    action_label_bits: int
    block_header_bits: int
    alignment_padding_bits: int
    reference_bits: int
    logical_effective_bits: float
    physical_effective_bits: float
    physical_compression_ratio: float

    @property
    def total_bits(self) -> int:
        return self.payload_bits + self.action_label_bits + self.block_header_bits + self.alignment_padding_bits

    def to_dict(self) -> dict[str, int | float]:
        out = asdict(self)
        out["total_bits"] = self.total_bits
        out["total_bytes"] = self.total_bits // 8
        return out


def _make_ledger(payload: int, labels: int, headers: int, padding: int, units: int, head_dim: int,
                 reference_bits: int) -> PackedLayoutLedger:
    scalars = 2 * units * int(head_dim)
    reference = scalars * int(reference_bits)
    total = payload + labels + headers + padding
    return PackedLayoutLedger(
        payload_bits=payload,
        action_label_bits=labels,
        block_header_bits=headers,
        alignment_padding_bits=padding,
        reference_bits=reference,
        logical_effective_bits=(payload + labels) / scalars,
        physical_effective_bits=total / scalars,
        physical_compression_ratio=reference / total,
    )


@dataclass(frozen=True)
class PackedNestedKVCache:
    """Packed K/V streams of one layer plus what block-local decoding needs."""

    key: PackedProgressiveStream
    value: PackedProgressiveStream
    action_labels: torch.Tensor
    mid_offsets: torch.Tensor
    high_offsets: torch.Tensor
    shape: tuple[int, int, int]
    head_dim: int
    stage_bits: tuple[int, ...]
    exits: tuple[int, int, int]
    block_size: int

    @property
    def units(self) -> int:
        b, h, t = self.shape
        return b * h * t

    @property
    def blocks_per_row(self) -> int:
        return _ceil_div(self.shape[-1], self.block_size)

    @property
    def block_count(self) -> int:
        return self.shape[0] * self.shape[1] * self.blocks_per_row

    @property
    def allocated_tensor_bytes(self) -> int:
        meta = (self.action_labels, self.mid_offsets, self.high_offsets)
        return (self.key.allocated_bytes + self.value.allocated_bytes
                + sum(int(t.numel() * t.element_size()) for t in meta))

    def ledger(self, *, reference_bits: int = 16) -> PackedLayoutLedger:
        """The cache's bits by kind; the total equals its allocated bytes
        (packed_nested.py:161-207)."""

        if reference_bits <= 0:
            raise ValueError("reference_bits must be positive")
        rates = prefix_index_bits(self.stage_bits, self.exits)
        depths = unpack_action_depths(self).to(torch.int64)
        payload = 2 * sum(int(depths.eq(d).sum()) * rates[d] for d in self.exits)
        labels = 2 * self.units
        headers = sum(int(o.numel() * o.element_size() * 8) for o in (self.mid_offsets, self.high_offsets))
        stream_bits = (self.key.allocated_bytes + self.value.allocated_bytes) * 8
        label_bits = int(self.action_labels.numel() * self.action_labels.element_size() * 8)
        padding = stream_bits - payload + label_bits - labels
        if padding < 0:
            raise RuntimeError("packed allocation is smaller than its logical fields")
        out = _make_ledger(payload, labels, headers, padding, self.units, self.head_dim, reference_bits)
        if out.total_bits != self.allocated_tensor_bytes * 8:
            raise RuntimeError("physical ledger differs from allocated tensor bytes")
        return out


# ---------------------------------------------------------------------------
# Layout arithmetic shared by the packer, the unpacker and the estimates


def _check_exits(schedule: tuple[int, ...], exits: Sequence[int]) -> tuple[int, int, int]:
    actions = tuple(int(d) for d in exits)
    if len(actions) != 3 or tuple(sorted(set(actions))) != actions:
        raise ValueError("exactly three sorted unique exits are required")
    if actions[0] <= 0 or actions[-1] > len(schedule):
        raise ValueError("exits must lie inside the stage schedule")
    return actions  # type: ignore[return-value]


def _check_depths_in_exits(depths: np.ndarray, actions: tuple[int, int, int], message: str) -> None:
    if not np.isin(depths, np.asarray(actions)).all():
        raise ValueError(message)


def _tier_ranges(actions: tuple[int, int, int]) -> tuple[tuple[int, int], ...]:
    return ((0, actions[0]), (actions[0], actions[1]), (actions[1], actions[2]))


def _blocked(depths_rt: np.ndarray, block_size: int) -> tuple[np.ndarray, np.ndarray]:
    """[rows, T] depths -> ([blocks, block_size] depths, real-token mask);
    blocks are row-major, padded tokens have depth 0 and mask False."""

    rows, tokens = depths_rt.shape
    per_row = _ceil_div(tokens, block_size)
    padded = np.zeros((rows, per_row * block_size), dtype=np.int64)
    padded[:, :tokens] = depths_rt
    real = np.zeros((rows, per_row * block_size), dtype=bool)
    real[:, :tokens] = True
    return padded.reshape(-1, block_size), real.reshape(-1, block_size)


def _tier_masks(block_depths: np.ndarray, real: np.ndarray, actions) -> tuple[np.ndarray, ...]:
    return (real, real & (block_depths >= actions[1]), real & (block_depths >= actions[2]))


def _segments(mask: np.ndarray, widths: Sequence[int]) -> tuple[np.ndarray, np.ndarray]:
    """Block offsets [blocks + 1] and (block, stage) segment starts of one tier."""

    counts = mask.sum(axis=1).astype(np.int64)
    w = np.asarray(widths, dtype=np.int64)
    seg = (counts[:, None] * w[None, :] + 7) // 8
    offsets = np.zeros(mask.shape[0] + 1, dtype=np.int64)
    np.cumsum(seg.sum(axis=1), out=offsets[1:])
    starts = offsets[:-1, None] + np.cumsum(seg, axis=1) - seg
    return offsets, starts


def _token_addresses(mask: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(block, slot) of every selected token in stream order and its rank."""

    rank = np.cumsum(mask, axis=1) - 1
    blk, slot = np.nonzero(mask)
    return blk, slot, rank[blk, slot]


def _pack_tier(indices: np.ndarray, mask: np.ndarray, stages: range, schedule) -> tuple[np.ndarray, np.ndarray]:
    widths = [schedule[s] for s in stages]
    offsets, starts = _segments(mask, widths)
    bits = np.zeros(int(offsets[-1]) * 8, dtype=np.uint8)
    blk, slot, rank = _token_addresses(mask)
    for k, s in enumerate(stages):
        w = widths[k]
        v = indices[blk, slot, s]
        if v.size and (v.min() < 0 or v.max() >= (1 << w)):
            raise ValueError(f"a value is outside the unsigned {w}-bit range")
        addr = starts[blk, k] * 8 + rank * w
        for j in range(w):
            bits[addr + j] = (v >> j) & 1
    return np.packbits(bits, bitorder="little"), offsets


def _unpack_tier(data: np.ndarray, mask: np.ndarray, stages: range, schedule, out: np.ndarray) -> None:
    widths = [schedule[s] for s in stages]
    _offsets, starts = _segments(mask, widths)
    bits = np.unpackbits(data, bitorder="little")
    blk, slot, rank = _token_addresses(mask)
    for k, s in enumerate(stages):
        w = widths[k]
        addr = starts[blk, k] * 8 + rank * w
        v = np.zeros(blk.size, dtype=np.int64)
        for j in range(w):
            v |= bits[addr + j].astype(np.int64) << j
        out[blk, slot, s] = v


# ---------------------------------------------------------------------------
# Packing, unpacking, validation


def _validate_layout_arguments(key_indices, value_indices, depths, *, stage_bits, exits, head_dim, block_size):
    schedule = validate_stage_bits(stage_bits)
    actions = _check_exits(schedule, exits)
    if key_indices.shape != value_indices.shape or key_indices.ndim != 4:
        raise ValueError("K/V indices must share [B,H,T,S] layout")
    if depths.shape != key_indices.shape[:-1]:
        raise ValueError("depths must have [B,H,T] layout")
    if key_indices.shape[-1] < actions[-1]:
        raise ValueError("indices do not contain the maximum exit")
    if head_dim <= 0 or block_size <= 0:
        raise ValueError("head_dim and block_size must be positive")
    local = depths.detach().to(device="cpu", dtype=torch.int64).numpy()
    _check_depths_in_exits(local, actions, "depth tensor contains an action outside the three exits")
    return schedule, actions, local


def _offset_tensor(offsets: np.ndarray) -> torch.Tensor:
    if int(offsets[-1]) > _INT32_MAX:
        raise ValueError("a per-layer stream exceeds the int32 offset range")
    return torch.from_numpy(offsets.astype(np.int32))


def _pack_kind(indices: torch.Tensor, block_depths, real, schedule, actions, block_size):
    b, h, t, s = indices.shape
    idx = indices.detach().to(device="cpu", dtype=torch.int64).reshape(b * h, t, s).numpy()
    per_row = _ceil_div(t, block_size)
    padded = np.zeros((b * h, per_row * block_size, s), dtype=np.int64)
    padded[:, :t] = idx
    padded = padded.reshape(-1, block_size, s)
    streams, offsets = [], []
    for mask, (first, last) in zip(_tier_masks(block_depths, real, actions), _tier_ranges(actions)):
        data, off = _pack_tier(padded, mask, range(first, last), schedule)
        streams.append(torch.from_numpy(data.copy()))
        offsets.append(off)
    return PackedProgressiveStream(*streams), offsets


def pack_paired_progressive_indices(
    key_indices: torch.Tensor,
    value_indices: torch.Tensor,
    depths: torch.Tensor,
    *,
    stage_bits: Sequence[int],
    exits: Sequence[int] = (14, 22, 30),
    head_dim: int = 128,
    block_size: int = 128,
) -> PackedNestedKVCache:
    """Pack one layer's K and V indices [B,H,T,S] at per-unit depths [B,H,T]
    into the progressive layout (packed_nested.py:547-601)."""

    schedule, actions, local = _validate_layout_arguments(
        key_indices, value_indices, depths, stage_bits=stage_bits, exits=exits, head_dim=head_dim,
        block_size=block_size)
    b, h, t = local.shape
    block_depths, real = _blocked(local.reshape(b * h, t), block_size)
    key, key_off = _pack_kind(key_indices, block_depths, real, schedule, actions, block_size)
    value, value_off = _pack_kind(value_indices, block_depths, real, schedule, actions, block_size)
    if any(not np.array_equal(a, c) for a, c in zip(key_off, value_off)):
        raise RuntimeError("paired K/V streams produced different block geometry")
    labels = np.searchsorted(np.asarray(actions), local.reshape(-1))
    cache = PackedNestedKVCache(
        key=key,
        value=value,
        action_labels=pack_fixed_width(torch.from_numpy(labels), 2),
        mid_offsets=_offset_tensor(key_off[1]),
        high_offsets=_offset_tensor(key_off[2]),
        shape=(int(b), int(h), int(t)),
        head_dim=int(head_dim),
        stage_bits=schedule,
        exits=actions,
        block_size=int(block_size),
    )
    validate_packed_nested_cache(cache)
    return cache


def unpack_action_depths(cache: PackedNestedKVCache) -> torch.Tensor:
    """Per-unit depths [B,H,T] (int16) from the 2-bit labels (:604-609)."""

    labels = unpack_fixed_width(cache.action_labels, 2, cache.units).to(torch.int64)
    if labels.numel() and int(labels.max()) >= len(cache.exits):
        raise ValueError("action map contains its reserved two-bit code")
    return torch.tensor(cache.exits, dtype=torch.int16)[labels].reshape(cache.shape)


def _unpack_kind(cache: PackedNestedKVCache, stream: PackedProgressiveStream, block_depths, real) -> torch.Tensor:
    b, h, t = cache.shape
    s = len(cache.stage_bits)
    out = np.zeros((block_depths.shape[0], cache.block_size, s), dtype=np.int64)
    stored = (None, cache.mid_offsets, cache.high_offsets)
    datas = (stream.base, stream.mid, stream.high)
    for tier, (mask, (first, last)) in enumerate(zip(_tier_masks(block_depths, real, cache.exits),
                                                     _tier_ranges(cache.exits))):
        widths = [cache.stage_bits[x] for x in range(first, last)]
        offsets, _ = _segments(mask, widths)
        if stored[tier] is not None and not np.array_equal(offsets, stored[tier].numpy().astype(np.int64)):
            raise ValueError("block offset does not match its packed stage segments")
        _unpack_tier(datas[tier].numpy(), mask, range(first, last), cache.stage_bits, out)
    out = out.reshape(b * h, -1, s)[:, :t]
    return torch.from_numpy(out.astype(np.uint8)).reshape(b, h, t, s)


def unpack_paired_progressive_indices(cache: PackedNestedKVCache) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Stored K and V indices [B,H,T,S] (uint8, zero past each unit's depth)
    and the depths [B,H,T] (:672-681)."""

    validate_packed_nested_cache(cache)
    depths = unpack_action_depths(cache)
    b, h, t = cache.shape
    block_depths, real = _blocked(depths.to(torch.int64).numpy().reshape(b * h, t), cache.block_size)
    key = _unpack_kind(cache, cache.key, block_depths, real)
    value = _unpack_kind(cache, cache.value, block_depths, real)
    return key, value, depths


def _base_offsets(cache: PackedNestedKVCache) -> np.ndarray:
    """Base-tier block offsets from the geometry alone (:612-623)."""

    b, h, t = cache.shape
    per_row = cache.blocks_per_row
    counts = np.full(per_row, cache.block_size, dtype=np.int64)
    counts[-1] = t - (per_row - 1) * cache.block_size
    w = np.asarray(cache.stage_bits[: cache.exits[0]], dtype=np.int64)
    per_block = ((counts[:, None] * w[None, :] + 7) // 8).sum(axis=1)
    offsets = np.zeros(b * h * per_row + 1, dtype=np.int64)
    np.cumsum(np.tile(per_block, b * h), out=offsets[1:])
    return offsets


def validate_packed_nested_cache(cache: PackedNestedKVCache) -> None:
    """Reject malformed streams before an unpack or a device hand-off
    (:684-734)."""

    if len(cache.shape) != 3 or any(v <= 0 for v in cache.shape):
        raise ValueError("shape must contain positive [B,H,T] dimensions")
    if cache.head_dim <= 0 or cache.block_size <= 0:
        raise ValueError("head_dim and block_size must be positive")
    validate_stage_bits(cache.stage_bits)
    ex = cache.exits
    if len(ex) != 3 or tuple(sorted(set(ex))) != tuple(ex) or ex[0] <= 0 or ex[-1] > len(cache.stage_bits):
        raise ValueError("cache exits are invalid")
    for t in (cache.key.base, cache.key.mid, cache.key.high, cache.value.base, cache.value.mid,
              cache.value.high, cache.action_labels):
        if t.device.type != "cpu" or t.dtype != torch.uint8 or t.ndim != 1:
            raise ValueError("packed byte streams must be flat CPU uint8 tensors")
    if cache.action_labels.numel() != _ceil_div(cache.units * 2, 8):
        raise ValueError("action-map byte length differs from the cache geometry")
    base_end = int(_base_offsets(cache)[-1])
    if base_end != cache.key.base.numel() or base_end != cache.value.base.numel():
        raise ValueError("derived base geometry differs from a paired stream size")
    for offsets, kd, vd in ((cache.mid_offsets, cache.key.mid, cache.value.mid),
                            (cache.high_offsets, cache.key.high, cache.value.high)):
        if (offsets.device.type != "cpu" or offsets.dtype != torch.int32 or offsets.ndim != 1
                or offsets.numel() != cache.block_count + 1):
            raise ValueError("block offsets must be flat CPU int32 tensors")
        o = offsets.to(torch.int64)
        if int(o[0]) != 0 or bool((o[1:] < o[:-1]).any()):
            raise ValueError("block offsets must be monotone and start at zero")
        if int(o[-1]) != kd.numel() or int(o[-1]) != vd.numel():
            raise ValueError("terminal block offset differs from a paired stream size")


# ---------------------------------------------------------------------------
# Byte estimates without packing


def estimate_paired_progressive_layout(
    depths: torch.Tensor,
    *,
    stage_bits: Sequence[int],
    exits: Sequence[int] = (14, 22, 30),
    head_dim: int = 128,
    block_size: int = 128,
    reference_bits: int = 16,
) -> PackedLayoutLedger:
    """The exact ledger :func:`pack_paired_progressive_indices` would produce
    for these depths, without any index payload (:210-309)."""

    schedule = validate_stage_bits(stage_bits)
    actions = _check_exits(schedule, exits)
    if depths.ndim != 3 or any(int(v) <= 0 for v in depths.shape):
        raise ValueError("depths must have positive [B,H,T] layout")
    if head_dim <= 0 or block_size <= 0 or reference_bits <= 0:
        raise ValueError("dimensions, block size, and reference width must be positive")
    local = depths.detach().to(device="cpu", dtype=torch.int64).numpy()
    _check_depths_in_exits(local, actions, "depth tensor contains an action outside the three exits")
    b, h, t = local.shape
    units = b * h * t
    rates = prefix_index_bits(schedule, actions)
    payload = 2 * sum(int((local == d).sum()) * rates[d] for d in actions)
    labels = 2 * units
    label_alloc = _ceil_div(labels, 8) * 8
    block_depths, real = _blocked(local.reshape(b * h, t), block_size)
    stream_bytes = 0
    for mask, (first, last) in zip(_tier_masks(block_depths, real, actions), _tier_ranges(actions)):
        offsets, _ = _segments(mask, schedule[first:last])
        stream_bytes += int(offsets[-1])
    stream_alloc = 2 * 8 * stream_bytes
    headers = 2 * (block_depths.shape[0] + 1) * 32
    padding = stream_alloc - payload + label_alloc - labels
    return _make_ledger(payload, labels, headers, padding, units, head_dim, reference_bits)


def estimate_layered_paired_progressive_layout(
    depths: torch.Tensor,
    *,
    stage_bits: Sequence[int],
    exits: Sequence[int] = (14, 22, 30),
    head_dim: int = 128,
    block_size: int = 128,
    reference_bits: int = 16,
) -> PackedLayoutLedger:
    """Sum of independent per-layer layouts for depths [L,B,H,T]: each layer
    has its own label stream and terminal offsets, so layers are byte-aligned
    separately (:312-365)."""

    if depths.ndim != 4 or any(int(v) <= 0 for v in depths.shape):
        raise ValueError("depths must have positive [L,B,H,T] layout")
    parts = [estimate_paired_progressive_layout(depths[layer], stage_bits=stage_bits, exits=exits,
                                                head_dim=head_dim, block_size=block_size,
                                                reference_bits=reference_bits)
             for layer in range(depths.shape[0])]
    payload = sum(p.payload_bits for p in parts)
    labels = sum(p.action_label_bits for p in parts)
    headers = sum(p.block_header_bits for p in parts)
    padding = sum(p.alignment_padding_bits for p in parts)
    return _make_ledger(payload, labels, headers, padding, int(depths.numel()), head_dim, reference_bits)


def estimate_block_shared_paired_progressive_layout(
    block_depths: torch.Tensor,
    token_counts: torch.Tensor,
    *,
    stage_bits: Sequence[int],
    exits: Sequence[int] = (14, 22, 30),
    head_dim: int = 128,
    reference_bits: int = 16,
) -> PackedLayoutLedger:
    """Ledger when one depth covers a token block: block depths [B,H,N],
    real tokens per block position [N]; one 2-bit label per block and one
    byte stream per K/V stage over the tokens that reach it, no offsets
    (:368-451)."""

    schedule = validate_stage_bits(stage_bits)
    actions = _check_exits(schedule, exits)
    if block_depths.ndim != 3 or any(int(v) <= 0 for v in block_depths.shape):
        raise ValueError("block depths must have positive [B,H,N_blocks] layout")
    if token_counts.ndim != 1 or token_counts.shape[0] != block_depths.shape[-1]:
        raise ValueError("token counts must have one entry per block position")
    if head_dim <= 0 or reference_bits <= 0:
        raise ValueError("head dimension and reference width must be positive")
    local = block_depths.detach().to(device="cpu", dtype=torch.int64).numpy()
    counts = token_counts.detach().to(device="cpu", dtype=torch.int64).numpy()
    if (counts <= 0).any():
        raise ValueError("every represented block must contain a real token")
    _check_depths_in_exits(local, actions, "block depth tensor contains an unknown action")
    weight = np.broadcast_to(counts, local.shape)
    units = int(weight.sum())
    rates = prefix_index_bits(schedule, actions)
    payload = 2 * sum(int(weight[local == d].sum()) * rates[d] for d in actions)
    one_kind = 0
    for stage, width in enumerate(schedule):
        active = int(weight[local > stage].sum())
        one_kind += _ceil_div(active * width, 8) * 8
    stream_alloc = 2 * one_kind
    blocks = local.size
    labels = 2 * blocks
    label_alloc = _ceil_div(labels, 8) * 8
    padding = stream_alloc - payload + label_alloc - labels
    if padding < 0:
        raise RuntimeError("block-shared allocation is smaller than its fields")
    return _make_ledger(payload, labels, 0, padding, units, head_dim, reference_bits)
