"""Rate ledger, prefix bit counts and fixed-width packing (host integers, CPU).

Every expected number here is worked out by hand in the comment beside it
(not by restating the formula), so a dropped K/V factor, a wrong position
width, a tail charged to the wrong side of the ratio or a reversed bit order
fails.  References: src/jointkv/budget.py:19-72 (CacheGeometry,
StorageLedger), :342-430 (residual_vq_ledger); src/jointkv/nested_vq.py:23-55
(stage bits, prefix_index_bits, paired_prefix_rates);
src/jointkv/packed_nested.py:30-72 (pack/unpack_fixed_width).
"""

from __future__ import annotations

import math

import pytest
import torch

from jointkv_amd import (
    CacheGeometry,
    ClosedLoopGroupedCQ,
    ClosedLoopUniformResidualVQ,
    StorageLedger,
    dynamic_bpa,
    pack_fixed_width,
    paired_prefix_rates,
    prefix_index_bits,
    residual_vq_ledger,
    unpack_fixed_width,
)

# 2 layers x 2 kv heads x 128 dims, a 100-token prompt, batch 1
SMALL = CacheGeometry(layers=2, kv_heads=2, head_dim=128, prompt_tokens=100)


def test_cache_geometry_scalars_and_validation():
    # K and V: 1 * 2 * 2 * 128 * 100 * 2 = 102,400 scalars
    assert SMALL.prompt_kv_scalars == 102_400
    # the Mistral-7B cache of the decode config: 32 * 8 * 128 * 4096 * 2 * 16 sequences
    mistral = CacheGeometry(layers=32, kv_heads=8, head_dim=128, prompt_tokens=4096, batch_size=16)
    assert mistral.prompt_kv_scalars == 4_294_967_296
    for bad in ({"layers": 0}, {"kv_heads": -1}, {"head_dim": 128.0}, {"reference_bits": 0}):
        args = dict(layers=2, kv_heads=2, head_dim=128, prompt_tokens=100)
        args.update(bad)
        with pytest.raises(ValueError, match="must be a positive integer"):
            CacheGeometry(**args)


def test_full_retention_g2_is_two_bits_per_scalar():
    # G2: 16 groups x 2 stages = 32 one-byte indices per head vector
    led = residual_vq_ledger(SMALL, retained_prompt_tokens=100, stages=32)
    assert isinstance(led, StorageLedger)
    # 1 * 2 layers * 2 heads * 100 tokens * 2 (K, V) = 800 vectors; 800 * 32 * 8 = 204,800 bits
    assert led.payload_bits == 204_800
    # no eviction: positions are implicit
    assert led.token_index_bits == 0
    assert led.fp16_tail_bits == 0
    assert led.affine_metadata_bits == led.control_metadata_bits == led.alignment_padding_bits == 0
    # 102,400 scalars * 16 bits
    assert led.reference_bits == 1_638_400
    assert led.total_bits == 204_800
    assert led.realized_effective_bits == 2.0
    assert led.nominal_effective_bits == 2.0
    assert led.compression_ratio == 8.0
    assert led.to_dict()["total_bits"] == 204_800
    # GSRQ1 / CQ1: 16 indices per vector = 1.0 bit per scalar
    one = residual_vq_ledger(SMALL, retained_prompt_tokens=100, stages=16)
    assert one.payload_bits == 102_400 and one.realized_effective_bits == 1.0


def test_eviction_charges_one_position_per_retained_pair():
    # 60 of 100 tokens kept: positions become explicit by default.
    # width = ceil(log2(100)) = 7 bits; per head: 2 layers * 2 heads * 60 * 7 = 1,680
    led = residual_vq_ledger(SMALL, retained_prompt_tokens=60, stages=32)
    assert led.token_index_bits == 1_680
    # 2 * 2 * 60 * 2 = 480 vectors * 256 bits = 122,880
    assert led.payload_bits == 122_880
    assert led.total_bits == 124_560
    # 124,560 / 102,400 scalars
    assert led.realized_effective_bits == pytest.approx(1.21640625, abs=0)
    # 0.6 * 32 * 8 / 128
    assert led.nominal_effective_bits == pytest.approx(1.2, rel=1e-15)
    assert led.compression_ratio == pytest.approx(1_638_400 / 124_560, rel=1e-15)
    # one position per layer shared by the heads: 2 * 1 * 60 * 7
    shared = residual_vq_ledger(SMALL, retained_prompt_tokens=60, stages=32, positions_per_head=False)
    assert shared.token_index_bits == 840
    # an explicit count of position-carrying tokens: 2 * 2 * 10 * 7
    some = residual_vq_ledger(SMALL, retained_prompt_tokens=60, stages=32, explicit_position_tokens=10)
    assert some.token_index_bits == 280
    # a 2-token prompt still needs a 1-bit position
    tiny = CacheGeometry(layers=1, kv_heads=1, head_dim=8, prompt_tokens=2)
    assert residual_vq_ledger(tiny, retained_prompt_tokens=1, stages=1).token_index_bits == 1
    # a power-of-two prompt: log2(4096) = 12 bits exactly
    p4k = CacheGeometry(layers=1, kv_heads=1, head_dim=128, prompt_tokens=4096)
    assert residual_vq_ledger(p4k, retained_prompt_tokens=4000, stages=1).token_index_bits == 4000 * 12


def test_fp16_tail_is_charged_and_referenced():
    # 5 decode tokens kept in fp16: 1 * 2 * 2 * 128 * 5 * 2 = 5,120 scalars -> 81,920 bits
    led = residual_vq_ledger(SMALL, retained_prompt_tokens=100, stages=32, fp16_decode_tokens=5)
    assert led.fp16_tail_bits == 81_920
    # the reference grows by the same scalars: (102,400 + 5,120) * 16
    assert led.reference_bits == 1_720_320
    assert led.total_bits == 204_800 + 81_920
    # 286,720 / 107,520 = 8/3; 1,720,320 / 286,720 = 6
    assert led.realized_effective_bits == pytest.approx(8 / 3, rel=1e-15)
    assert led.compression_ratio == 6.0


def test_ledger_error_texts():
    with pytest.raises(ValueError, match="retained_prompt_tokens must be within the prompt"):
        residual_vq_ledger(SMALL, retained_prompt_tokens=0, stages=2)
    with pytest.raises(ValueError, match="retained_prompt_tokens must be within the prompt"):
        residual_vq_ledger(SMALL, retained_prompt_tokens=101, stages=2)
    with pytest.raises(ValueError, match="VQ stage and code widths must be positive"):
        residual_vq_ledger(SMALL, retained_prompt_tokens=10, stages=0)
    with pytest.raises(ValueError, match="VQ stage and code widths must be positive"):
        residual_vq_ledger(SMALL, retained_prompt_tokens=10, stages=2, codebook_bits=0)
    with pytest.raises(ValueError, match="fp16_decode_tokens cannot be negative"):
        residual_vq_ledger(SMALL, retained_prompt_tokens=10, stages=2, fp16_decode_tokens=-1)
    with pytest.raises(ValueError, match="explicit_position_tokens is outside retained tokens"):
        residual_vq_ledger(SMALL, retained_prompt_tokens=10, stages=2, explicit_position_tokens=11)


def test_prefix_index_bits_and_paired_rates():
    # schedule 8, 8, 4, 2 bits: prefixes 1, 3, 4 carry 8, 8+8+4 = 20, 22 bits
    assert prefix_index_bits([8, 8, 4, 2], [4, 1, 3, 3]) == {1: 8, 3: 20, 4: 22}
    # K and V: twice each
    assert paired_prefix_rates([8, 8, 4, 2], [1, 3, 4]) == {1: 16, 3: 40, 4: 44}
    # the G2 ladder: 32 one-byte indices, exits at 16 and 32 indices
    assert prefix_index_bits([8] * 32, [16, 32]) == {16: 128, 32: 256}
    for bad in ([0, 8], [9], []):
        with pytest.raises(ValueError, match="stage bits must lie in"):
            prefix_index_bits(bad, [1])
    for bad in ([0], [5], []):
        with pytest.raises(ValueError, match="prefixes must lie inside the stage schedule"):
            prefix_index_bits([8, 8, 4, 2], bad)


def test_dynamic_bpa_and_codec_rates():
    # 16 one-byte indices over 128 dims = 1.0; 32 = 2.0; 32 four-bit indices = 1.0
    assert dynamic_bpa(16, 128) == 1.0
    assert dynamic_bpa(32, 128) == 2.0
    assert dynamic_bpa(32, 128, bits=4) == 1.0
    with pytest.raises(ValueError):
        dynamic_bpa(0, 128)
    # the codecs keep the rate they are built with (uniform_depth_tac.py:64, cq_tac.py:159)
    tables = [torch.zeros(2, 16, 2, 256, 8)]
    codec = ClosedLoopUniformResidualVQ(tables, tables, [None], depth=2, dynamic_bpa=dynamic_bpa(32, 128))
    assert codec.dynamic_bpa == 2.0
    books = [torch.zeros(2, 32, 256, 4)]
    eye = [torch.eye(4).repeat(2, 32, 1, 1)]
    cq = ClosedLoopGroupedCQ(books, books, eye, dynamic_bpa=dynamic_bpa(32, 128))
    assert cq.dynamic_bpa == 2.0


# ---------------------------------------------------------------------------
# LSB-first fixed-width packing


@pytest.mark.parametrize(
    "values,width,expect",
    [
        # 1-bit: bits 1,0,1,1,0,0,0,1 | 1 -> 1+4+8+128 = 141, then 1
        ([1, 0, 1, 1, 0, 0, 0, 1, 1], 1, [141, 1]),
        # 3-bit: 5 -> 1,0,1; 3 -> 1,1,0; 7 -> 1,1,1; 1 -> 1,0,0
        # byte 0 = 1,0,1,1,1,0,1,1 = 1+4+8+16+64+128 = 221; byte 1 = 1,1,0,0 = 3
        ([5, 3, 7, 1], 3, [221, 3]),
        # 5-bit: 31 -> 1,1,1,1,1; 0 -> 0,0,0,0,0; 17 -> 1,0,0,0,1
        # byte 0 = 1,1,1,1,1,0,0,0 = 31; byte 1 = 0,0,1,0,0,0,1,0 = 4+64 = 68
        ([31, 0, 17], 5, [31, 68]),
        # 4-bit: low nibble first: (0xA, 0x5) -> 0x5A; (0xF, 0x1) -> 0x1F
        ([10, 5, 15, 1], 4, [0x5A, 0x1F]),
        # 8-bit: identity
        ([0, 255, 17], 8, [0, 255, 17]),
    ],
)
def test_pack_fixed_width_byte_layout(values, width, expect):
    packed = pack_fixed_width(torch.tensor(values), width)
    assert packed.dtype == torch.uint8
    assert packed.tolist() == expect
    back = unpack_fixed_width(packed, width, len(values))
    assert back.tolist() == values


@pytest.mark.parametrize("width", range(1, 9))
@pytest.mark.parametrize("count", [0, 1, 7, 8, 9, 1000, 1003])
def test_pack_round_trip_every_width(width, count):
    gen = torch.Generator().manual_seed(100 * width + count)
    values = torch.randint(0, 1 << width, (count,), generator=gen)
    packed = pack_fixed_width(values, width)
    assert packed.numel() == math.ceil(count * width / 8)
    assert torch.equal(unpack_fixed_width(packed, width, count), values.to(torch.uint8))
    # every bit of the stream lands where LSB-first order puts it
    if count:
        bits = [(int(v) >> i) & 1 for v in values for i in range(width)]
        bits += [0] * (-len(bits) % 8)
        expect = [sum(bits[8 * j + i] << i for i in range(8)) for j in range(len(bits) // 8)]
        assert packed.tolist() == expect


def test_pack_rejects_bad_widths_and_ranges():
    with pytest.raises(ValueError, match="bits must lie in"):
        pack_fixed_width(torch.tensor([1]), 0)
    with pytest.raises(ValueError, match="bits must lie in"):
        pack_fixed_width(torch.tensor([1]), 9)
    with pytest.raises(ValueError, match="outside the unsigned 3-bit range"):
        pack_fixed_width(torch.tensor([8]), 3)
    with pytest.raises(ValueError, match="outside the unsigned 3-bit range"):
        pack_fixed_width(torch.tensor([-1]), 3)
    with pytest.raises(ValueError, match="expected 2"):
        unpack_fixed_width(torch.zeros(3, dtype=torch.uint8), 3, 4)
    with pytest.raises(ValueError, match="count must be non-negative"):
        unpack_fixed_width(torch.zeros(0, dtype=torch.uint8), 3, -1)
