"""Paired progressive code streams and their ledgers (host only, CPU).

The vectorised packer in jointkv_amd.packed_nested against the loop oracle
(oracle/packed_nested_oracle.py), which a hand-worked layout pins.
"""

from __future__ import annotations

import pytest
import torch

from jointkv_amd import packed_nested as pn
from oracle import packed_nested_oracle as po

# three tokens, block size 2, stage widths (2, 3, 1), exits (1, 2, 3)
HAND_DEPTHS = [[[1, 3, 2]]]
HAND_KEY = [[[[3, 5, 1], [1, 7, 1], [2, 4, 0]]]]


def test_oracle_hand_worked_layout():
    # base (stage 0, 2 bits, all tokens): block 0 holds 3, 1 -> bits 11 10 ->
    # 0b0111; block 1 holds 2 -> bits 01 -> 0b10.  mid (stage 1, 3 bits, depth
    # >= 2): block 0 token 1 -> 7; block 1 token 2 -> 4.  high (stage 2, 1 bit,
    # depth 3): block 0 token 1 -> 1; block 1 empty.
    data, offsets = po.pack_stream(HAND_KEY, HAND_DEPTHS, (2, 3, 1), (1, 2, 3), 2)
    assert data == [[7, 2], [7, 4], [1]]
    assert offsets == [[0, 1, 2], [0, 1, 2], [0, 1, 1]]
    # labels 0, 2, 1 at 2 bits LSB first: 00 01 10 -> 0b011000
    assert po.action_labels(HAND_DEPTHS, (1, 2, 3)) == [24]
    back = po.unpack_stream(data, HAND_DEPTHS, (2, 3, 1), (1, 2, 3), 2, 3)
    assert back == [[[[3, 0, 0], [1, 7, 1], [2, 4, 0]]]]
    # payload 2 * (2 + 6 + 5) = 26, labels 6, headers 2 * 3 * 32 = 192,
    # padding 2 * 5 * 8 - 26 + 8 - 6 = 56: 280 bits = 35 allocated bytes
    assert po.ledger_bits(HAND_DEPTHS, (2, 3, 1), (1, 2, 3), 5, 1, 2) == (26, 6, 192, 56)


def test_packer_matches_the_hand_worked_layout():
    key = torch.tensor(HAND_KEY)
    cache = pn.pack_paired_progressive_indices(key, key.flip(-1) % 2, torch.tensor(HAND_DEPTHS),
                                               stage_bits=(2, 3, 1), exits=(1, 2, 3), head_dim=4, block_size=2)
    assert cache.key.base.tolist() == [7, 2] and cache.key.mid.tolist() == [7, 4] and cache.key.high.tolist() == [1]
    assert cache.mid_offsets.tolist() == [0, 1, 2] and cache.high_offsets.tolist() == [0, 1, 1]
    assert cache.mid_offsets.dtype == torch.int32 and cache.action_labels.tolist() == [24]
    led = cache.ledger()
    assert (led.payload_bits, led.action_label_bits, led.block_header_bits, led.alignment_padding_bits) == (
        26, 6, 192, 56)
    assert led.total_bits == 280 == cache.allocated_tensor_bytes * 8
    assert led.reference_bits == 2 * 3 * 4 * 16
    assert led.to_dict()["total_bytes"] == 35
    k, v, d = pn.unpack_paired_progressive_indices(cache)
    assert k.tolist() == [[[[3, 0, 0], [1, 7, 1], [2, 4, 0]]]]
    assert d.dtype == torch.int16 and d.tolist() == HAND_DEPTHS


def _random_layer(seed, shape, stage_bits, exits):
    gen = torch.Generator().manual_seed(seed)
    s = len(stage_bits)
    hi = torch.tensor([1 << w for w in stage_bits])
    key = (torch.rand(*shape, s, generator=gen) * hi).long()
    value = (torch.rand(*shape, s, generator=gen) * hi).long()
    depths = torch.tensor(exits)[torch.randint(0, 3, shape, generator=gen)]
    return key, value, depths


@pytest.mark.parametrize("seed,shape,stage_bits,exits,block", [
    (0, (1, 2, 9), (2, 3, 1, 8, 5), (1, 3, 5), 4),
    (1, (2, 3, 37), (8,) * 6, (2, 4, 6), 16),
    (2, (1, 1, 128), (3, 5, 7, 1, 2, 8, 4, 6), (2, 5, 8), 128),
    (3, (2, 2, 130), (4,) * 30, (14, 22, 30), 128),
])
def test_packer_bytes_equal_the_oracle(seed, shape, stage_bits, exits, block):
    key, value, depths = _random_layer(seed, shape, stage_bits, exits)
    cache = pn.pack_paired_progressive_indices(key, value, depths, stage_bits=stage_bits, exits=exits,
                                               block_size=block)
    for kind, idx in (("key", key), ("value", value)):
        data, offsets = po.pack_stream(idx.tolist(), depths.tolist(), stage_bits, exits, block)
        stream = getattr(cache, kind)
        assert [stream.base.tolist(), stream.mid.tolist(), stream.high.tolist()] == data
    assert cache.mid_offsets.tolist() == offsets[1] and cache.high_offsets.tolist() == offsets[2]
    assert cache.action_labels.tolist() == po.action_labels(depths.tolist(), exits)
    # round trip: stored stages come back, the rest are zero
    k, v, d = pn.unpack_paired_progressive_indices(cache)
    keep = torch.arange(len(stage_bits)) < depths[..., None]
    assert torch.equal(k.long(), key * keep) and torch.equal(v.long(), value * keep)
    assert torch.equal(d.long(), depths)
    # the ledger totals the allocated bytes; the estimate predicts it exactly
    led = cache.ledger()
    assert led.total_bits == cache.allocated_tensor_bytes * 8
    assert (led.payload_bits, led.action_label_bits, led.block_header_bits, led.alignment_padding_bits) == (
        po.ledger_bits(depths.tolist(), stage_bits, exits, cache.key.allocated_bytes,
                       cache.action_labels.numel(), cache.block_count))
    assert pn.estimate_paired_progressive_layout(depths, stage_bits=stage_bits, exits=exits,
                                                 block_size=block) == led


def test_layered_estimate_sums_byte_aligned_layers():
    stage_bits, exits = (3, 5, 2, 7), (1, 2, 4)
    layers = [_random_layer(10 + i, (1, 2, 21), stage_bits, exits)[2] for i in range(3)]
    total = pn.estimate_layered_paired_progressive_layout(torch.stack(layers), stage_bits=stage_bits, exits=exits,
                                                          block_size=8)
    parts = [pn.pack_paired_progressive_indices(*_random_layer(10 + i, (1, 2, 21), stage_bits, exits),
                                                stage_bits=stage_bits, exits=exits, block_size=8)
             for i in range(3)]
    assert total.total_bits == sum(p.allocated_tensor_bytes * 8 for p in parts)
    assert total.payload_bits == sum(p.ledger().payload_bits for p in parts)


def test_block_shared_estimate_hand_worked():
    # one row, blocks of 2 and 1 real tokens at depths 1 and 3, widths (2,3,1):
    # payload 2 (2*2 + 1*6) = 20; stage streams over 3, 1, 1 tokens -> 6, 3, 1
    # bits -> one byte each, 48 bits for K+V; 2 labels -> one byte; padding
    # 48 - 20 + 8 - 4 = 32
    led = pn.estimate_block_shared_paired_progressive_layout(
        torch.tensor([[[1, 3]]]), torch.tensor([2, 1]), stage_bits=(2, 3, 1), exits=(1, 2, 3), head_dim=4)
    assert (led.payload_bits, led.action_label_bits, led.block_header_bits, led.alignment_padding_bits) == (
        20, 4, 0, 32)
    assert led.reference_bits == 2 * 3 * 4 * 16 and led.total_bits == 56


def test_errors_match_the_reference_texts():
    key, value, depths = _random_layer(5, (1, 1, 8), (2, 2, 2), (1, 2, 3))
    kw = dict(stage_bits=(2, 2, 2), block_size=4)
    with pytest.raises(ValueError, match="exactly three sorted unique exits"):
        pn.pack_paired_progressive_indices(key, value, depths, exits=(2, 1, 3), **kw)
    with pytest.raises(ValueError, match="outside the three exits"):
        pn.pack_paired_progressive_indices(key, value, depths.clone().fill_(2).index_fill_(-1, torch.tensor([0]), 0),
                                           exits=(1, 2, 3), **kw)
    with pytest.raises(ValueError, match="outside the unsigned 2-bit range"):
        pn.pack_paired_progressive_indices(key.clone().fill_(4), value, depths, exits=(1, 2, 3), **kw)
    with pytest.raises(ValueError, match="maximum exit"):
        pn.pack_paired_progressive_indices(key[..., :2], value[..., :2], depths, exits=(1, 2, 3), **kw)
    cache = pn.pack_paired_progressive_indices(key, value, depths, exits=(1, 2, 3), **kw)
    bad = pn.PackedNestedKVCache(**{**cache.__dict__, "mid_offsets": cache.mid_offsets.long()})
    with pytest.raises(ValueError, match="flat CPU int32"):
        pn.unpack_paired_progressive_indices(bad)
    # offsets that keep the terminal size but move a block boundary
    moved = cache.mid_offsets.clone()
    if moved.numel() > 2 and moved[1] > 0:
        moved[1] -= 1
        bad = pn.PackedNestedKVCache(**{**cache.__dict__, "mid_offsets": moved})
        with pytest.raises(ValueError, match="block offset does not match"):
            pn.unpack_paired_progressive_indices(bad)
    labels = cache.action_labels.clone()
    labels[0] = 0xFF
    with pytest.raises(ValueError, match="reserved two-bit code"):
        pn.unpack_action_depths(pn.PackedNestedKVCache(**{**cache.__dict__, "action_labels": labels}))
