"""CPU oracle for the paired progressive code-stream layout.

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` may import this module, as the
checker of ``jointkv_amd.packed_nested``; the product never calls it.

A scalar restatement, in plain Python loops over blocks, stages and bits, of
src/jointkv/packed_nested.py: LSB-first fixed-width packing (:30-47), the
per-block tier walk of ``_pack_stream`` (:494-538) and ``_unpack_stream``
(:626-669), the 2-bit action labels (:589-593, :604-609) and the ledger
arithmetic of ``PackedNestedKVCache.ledger`` (:161-207).  Small inputs only.

Pins (tests/test_packed_nested.py): a hand-worked three-token layout with
its bytes, offsets, labels and ledger written out; round trips; the
reference's own invariant that a cache's ledger totals its allocated bytes.
"""

from __future__ import annotations


def pack_bits(values, width):
    """LSB-first: value i fills bits [i*width, (i+1)*width); bytes zero-padded."""

    out = bytearray((len(values) * width + 7) // 8)
    pos = 0
    for v in values:
        for j in range(width):
            if (v >> j) & 1:
                out[pos >> 3] |= 1 << (pos & 7)
            pos += 1
    return list(out)


def unpack_bits(data, width, count):
    vals = []
    pos = 0
    for _ in range(count):
        v = 0
        for j in range(width):
            v |= ((data[pos >> 3] >> (pos & 7)) & 1) << j
            pos += 1
        vals.append(v)
    return vals


def _blocks(shape, block_size):
    b, h, t = shape
    for row in range(b * h):
        for start in range(0, t, block_size):
            yield row, start, min(t, start + block_size)


def pack_stream(indices, depths, stage_bits, exits, block_size):
    """indices: nested lists [B][H][T][S]; depths [B][H][T].  Returns the three
    tier byte lists and their block offsets (base offsets included)."""

    b, h, t = len(depths), len(depths[0]), len(depths[0][0])
    flat_idx = [indices[i][j] for i in range(b) for j in range(h)]
    flat_dep = [depths[i][j] for i in range(b) for j in range(h)]
    tiers = ((0, exits[0], 0), (exits[0], exits[1], exits[1]), (exits[1], exits[2], exits[2]))
    data = [[], [], []]
    offsets = [[0], [0], [0]]
    for row, start, stop in _blocks((b, h, t), block_size):
        for k, (first, last, need) in enumerate(tiers):
            chosen = [tok for tok in range(start, stop) if flat_dep[row][tok] >= need]
            for stage in range(first, last):
                data[k] += pack_bits([flat_idx[row][tok][stage] for tok in chosen], stage_bits[stage])
            offsets[k].append(len(data[k]))
    return data, offsets


def unpack_stream(data, depths, stage_bits, exits, block_size, stages):
    b, h, t = len(depths), len(depths[0]), len(depths[0][0])
    flat_dep = [depths[i][j] for i in range(b) for j in range(h)]
    out = [[[0] * stages for _ in range(t)] for _ in range(b * h)]
    tiers = ((0, exits[0], 0), (exits[0], exits[1], exits[1]), (exits[1], exits[2], exits[2]))
    cursor = [0, 0, 0]
    for row, start, stop in _blocks((b, h, t), block_size):
        for k, (first, last, need) in enumerate(tiers):
            chosen = [tok for tok in range(start, stop) if flat_dep[row][tok] >= need]
            for stage in range(first, last):
                nbytes = (len(chosen) * stage_bits[stage] + 7) // 8
                vals = unpack_bits(data[k][cursor[k]:cursor[k] + nbytes], stage_bits[stage], len(chosen))
                for tok, v in zip(chosen, vals):
                    out[row][tok][stage] = v
                cursor[k] += nbytes
    return [[out[i * h + j] for j in range(h)] for i in range(b)]


def action_labels(depths, exits):
    flat = [d for plane in depths for row in plane for d in row]
    return pack_bits([exits.index(d) for d in flat], 2)


def ledger_bits(depths, stage_bits, exits, stream_bytes, label_bytes, block_count):
    """(payload, labels, headers, padding) bits of one paired K/V cache whose
    K and V streams hold ``stream_bytes`` bytes each."""

    flat = [d for plane in depths for row in plane for d in row]
    rate = {d: sum(stage_bits[:d]) for d in exits}
    payload = 2 * sum(rate[d] for d in flat)
    labels = 2 * len(flat)
    headers = 2 * (block_count + 1) * 32
    padding = 2 * stream_bytes * 8 - payload + label_bytes * 8 - labels
    return payload, labels, headers, padding
