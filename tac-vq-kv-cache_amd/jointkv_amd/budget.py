"""Rate ledger of the per-token residual-VQ code cache (host-side integers).

Keeps the reference's accounting (src/jointkv/budget.py: ``CacheGeometry``
:19-42, ``StorageLedger`` :45-72, ``residual_vq_ledger`` :342-430) and the
fixed-width prefix bit counts of src/jointkv/nested_vq.py:23-55, so that a
request's cache bytes and bits-per-scalar read the same here as there:
payload = one ``codebook_bits`` index per stage per retained K and V head
vector; explicit positions when eviction makes them non-contiguous; an
optional fp16 decode tail; codebooks are model-static and excluded.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from math import ceil, log2
from typing import Iterable, Sequence


@dataclass(frozen=True)
class CacheGeometry:
    layers: int
    kv_heads: int
    head_dim: int
    prompt_tokens: int
    batch_size: int = 1
    reference_bits: int = 16

    def __post_init__(self) -> None:
        for name, value in asdict(self).items():
            if not isinstance(value, int) or value <= 0:
                raise ValueError(f"{name} must be a positive integer, got {value!r}")

    @property
    def prompt_kv_scalars(self) -> int:
        return self.batch_size * self.layers * self.kv_heads * self.head_dim * self.prompt_tokens * 2


@dataclass(frozen=True)
class StorageLedger:
    payload_bits: int
    affine_metadata_bits: int
    token_index_bits: int
    control_metadata_bits: int
    alignment_padding_bits: int
    fp16_tail_bits: int
    reference_bits: int
    nominal_effective_bits: float
    realized_effective_bits: float
    compression_ratio: float

    @property
    def total_bits(self) -> int:
        return (
            self.payload_bits
            + self.affine_metadata_bits
            + self.token_index_bits
            + self.control_metadata_bits
            + self.alignment_padding_bits
            + self.fp16_tail_bits
        )

    def to_dict(self) -> dict[str, int | float]:
        out = asdict(self)
        out["total_bits"] = self.total_bits
        return out


def residual_vq_ledger(
    geometry: CacheGeometry,
    *,
    retained_prompt_tokens: int,
    stages: int,
    codebook_bits: int = 8,
    explicit_position_tokens: int | None = None,
    positions_per_head: bool = True,
    fp16_decode_tokens: int = 0,
) -> StorageLedger:
    """Dynamic-cache ledger for a per-token residual VQ (budget.py:342-430)."""

    g = geometry
    if not 0 < retained_prompt_tokens <= g.prompt_tokens:
        raise ValueError("retained_prompt_tokens must be within the prompt")
    if stages <= 0 or codebook_bits <= 0:
        raise ValueError("VQ stage and code widths must be positive")
    if fp16_decode_tokens < 0:
        raise ValueError("fp16_decode_tokens cannot be negative")
    if explicit_position_tokens is None:
        explicit_position_tokens = retained_prompt_tokens if retained_prompt_tokens < g.prompt_tokens else 0
    if not 0 <= explicit_position_tokens <= retained_prompt_tokens:
        raise ValueError("explicit_position_tokens is outside retained tokens")
    per_layer_heads = g.batch_size * g.layers * g.kv_heads
    payload = per_layer_heads * retained_prompt_tokens * 2 * stages * codebook_bits
    width = max(1, ceil(log2(max(2, g.prompt_tokens))))
    position_heads = g.kv_heads if positions_per_head else 1
    token_index = g.batch_size * g.layers * position_heads * explicit_position_tokens * width
    tail_scalars = per_layer_heads * g.head_dim * fp16_decode_tokens * 2
    tail = tail_scalars * g.reference_bits
    reference_scalars = g.prompt_kv_scalars + tail_scalars
    reference = reference_scalars * g.reference_bits
    total = payload + token_index + tail
    return StorageLedger(
        payload_bits=payload,
        affine_metadata_bits=0,
        token_index_bits=token_index,
        control_metadata_bits=0,
        alignment_padding_bits=0,
        fp16_tail_bits=tail,
        reference_bits=reference,
        nominal_effective_bits=retained_prompt_tokens / g.prompt_tokens * stages * codebook_bits / g.head_dim,
        realized_effective_bits=total / reference_scalars,
        compression_ratio=reference / total,
    )


def validate_stage_bits(stage_bits: Sequence[int]) -> tuple[int, ...]:
    """Fixed-width stage index widths, each in [1, 8] (nested_vq.py:23-29)."""

    widths = tuple(int(b) for b in stage_bits)
    if not widths or any(b <= 0 or b > 8 for b in widths):
        raise ValueError("stage bits must lie in [1, 8]")
    return widths


def prefix_index_bits(stage_bits: Sequence[int], prefixes: Iterable[int]) -> dict[int, int]:
    """Cumulative index bits per vector at each requested prefix (nested_vq.py:32-46)."""

    widths = validate_stage_bits(stage_bits)
    wanted = sorted({int(p) for p in prefixes})
    if not wanted or wanted[0] <= 0 or wanted[-1] > len(widths):
        raise ValueError("prefixes must lie inside the stage schedule")
    out: dict[int, int] = {}
    running = 0
    for depth, width in enumerate(widths, start=1):
        running += width
        if depth in wanted:
            out[depth] = running
    return out


def paired_prefix_rates(stage_bits: Sequence[int], prefixes: Iterable[int]) -> dict[int, int]:
    """K+V payload bits per token/head pair at each prefix (nested_vq.py:49-55)."""

    return {depth: 2 * bits for depth, bits in prefix_index_bits(stage_bits, prefixes).items()}


def dynamic_bpa(index_count: int, head_dim: int, bits: int = 8) -> float:
    """Bits per cached scalar of a code with ``index_count`` fixed-width indices."""

    if index_count <= 0 or head_dim <= 0 or bits <= 0:
        raise ValueError("index count, head dim and width must be positive")
    return index_count * bits / head_dim
