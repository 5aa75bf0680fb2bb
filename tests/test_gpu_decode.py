"""Fused decode attention over packed code caches vs the oracle's
decode -> RoPE -> repeat_kv -> SDPA sequence (2e-3 max abs)."""

from __future__ import annotations

import pytest
import torch

import jointkv_amd as jkv
from oracle import jointkv_oracle as ref
from parity import compare_codes

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def _case(seed, batch, qh, kvh, groups, stages, d, length, cap):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, qh, 1, 128, generator=gen).half()
    kc = torch.randint(0, 256, (batch, kvh, cap, groups, stages), generator=gen, dtype=torch.uint8)
    vc = torch.randint(0, 256, (batch, kvh, cap, groups, stages), generator=gen, dtype=torch.uint8)
    sig = (1.0, 0.5, 0.25, 0.125)[:stages] if stages <= 4 else tuple(0.8 ** s for s in range(stages))
    kt = ref.synthetic_tables(gen, (kvh * groups, stages, 256, d), sig, stage_axis=1)
    vt = ref.synthetic_tables(gen, (kvh * groups, stages, 256, d), sig, stage_axis=1)
    return q, kc, vc, kt, vt


def _expect(q, kc, vc, kt, vt, length, window, cap):
    start = max(0, length - window)
    pos = torch.arange(start, length)
    slots = pos % cap
    khat = ref.frozen_decode(kc[:, :, slots].contiguous(), kt, kt.shape[1], torch.float16)
    vhat = ref.frozen_decode(vc[:, :, slots].contiguous(), vt, vt.shape[1], torch.float16)
    return ref.decode_attention(q, khat, vhat, length - 1, pos)


@pytest.mark.parametrize("batch,qh,kvh,groups,stages,d,length,window,cap", [
    (2, 32, 8, 16, 2, 8, 4096, 4096, 4096),   # config 4 geometry, full window
    (16, 32, 8, 16, 2, 8, 4096, 4096, 4096),  # config 4 exactly: batch 16 (the benchmarked block mapping)
    (1, 8, 2, 16, 2, 8, 300, 4096, 4096),     # short prefix
    (1, 8, 2, 16, 2, 8, 5000, 4096, 4096),    # window slides, ring buffer wraps
    (1, 4, 4, 32, 1, 4, 700, 512, 512),       # cq2 codes, MHA group of 1
    (1, 16, 2, 16, 1, 8, 257, 4096, 4096),    # cq1 codes, GQA 8
    (1, 2, 2, 16, 2, 8, 1000, 4096, 4096),    # one query head per kv head at d = 8
    (2, 4, 2, 16, 1, 8, 1500, 512, 1024),     # GQA 2, one stage, window of two 256-token chunks, ring wraps
    (1, 8, 2, 16, 3, 8, 600, 4096, 4096),     # three stages: the generic split kernel
    (1, 8, 2, 1, 4, 128, 600, 4096, 4096),    # full-vector codebooks, 4 stages (codewords from L2)
    (2, 32, 8, 1, 16, 128, 700, 256, 512),    # full-vector R16 geometry, sliding window, ring wraps
    (1, 16, 2, 1, 16, 128, 300, 4096, 512),   # R16 codes, GQA 8
    (1, 8, 2, 1, 32, 128, 333, 4096, 512),    # R32 codes, ragged last tile
    (1, 2, 2, 1, 32, 128, 170, 4096, 256),    # R32 codes, one query head per kv head
])
def test_decode_matches_oracle(device, batch, qh, kvh, groups, stages, d, length, window, cap):
    q, kc, vc, kt, vt = _case(length + qh, batch, qh, kvh, groups, stages, d, length, cap)
    print(f"decode B={batch} QH={qh} KVH={kvh} G={groups} S={stages} len={length} win={window}", flush=True)
    out = jkv.decode_attention(
        q.to(device), kc.to(device), vc.to(device), kt.half().to(device), vt.half().to(device),
        torch.full((batch,), length, dtype=torch.int32, device=device), window=window,
    )
    expect = _expect(q, kc, vc, kt, vt, length, window, cap)
    err = float((out.cpu().float() - expect.float()).abs().max())
    assert err <= ATOL, f"max abs error {err}"


@pytest.mark.parametrize("batch,qh,kvh,stages,lengths,window,cap", [
    (2, 32, 8, 2, (4096, 4096), 4096, 4096),    # config 4 geometry: the new token closes split 2
    (3, 8, 2, 2, (1, 257, 5000), 4096, 4096),   # first token; chunk 1's first key; ring wrap
    (2, 16, 2, 1, (600, 2049), 4096, 4096),     # one stage, GQA 8; the new token opens split 2
    (2, 4, 2, 2, (513, 700), 512, 1024),        # window of two chunks, partial last chunk
    (16, 32, 8, 2, (4096,) * 16, 4096, 4096),   # config 4 exactly: batch 16, the benchmarked grid
])
def test_decode_append_matches_encode_then_decode(device, batch, qh, kvh, stages, lengths, window, cap):
    # the fused step encodes the new token into its slot and attends with it
    print(f"decode append B={batch} QH={qh} KVH={kvh} S={stages} lengths={lengths} win={window}", flush=True)
    q, kc, vc, kt, vt = _case(sum(lengths) + qh, batch, qh, kvh, 16, stages, 8, 0, cap)
    gen = torch.Generator().manual_seed(4242 + sum(lengths))
    knew = ref.synthetic_states(gen, batch, kvh, 1)
    vnew = ref.synthetic_states(gen, batch, kvh, 1)
    lens = torch.tensor(lengths, dtype=torch.int32)
    kc_d, vc_d = kc.to(device), vc.to(device)
    kt16, vt16 = kt.half().to(device), vt.half().to(device)
    out = jkv.decode_attention(q.to(device), kc_d, vc_d, kt16, vt16, lens.to(device), window=window,
                               key_new=knew.to(device), value_new=vnew.to(device))
    kc_got, vc_got = kc_d.cpu(), vc_d.cpu()
    slots = [(int(L) - 1) % cap for L in lengths]
    # only the new tokens' slots changed
    keep = torch.ones(batch, cap, dtype=torch.bool)
    for b, sl in enumerate(slots):
        keep[b, sl] = False
    assert torch.equal(kc_got.permute(0, 2, 1, 3, 4)[keep], kc.permute(0, 2, 1, 3, 4)[keep])
    assert torch.equal(vc_got.permute(0, 2, 1, 3, 4)[keep], vc.permute(0, 2, 1, 3, 4)[keep])
    # the written codes are the codec's greedy search of the raw vectors
    for raw, tabs, got in ((knew, kt, kc_got), (vnew, vt, vc_got)):
        _o, want, d1, d2 = ref.grouped_residual_vq(raw, tabs.reshape(kvh, 16, stages, 256, 8), prefixes=(stages,),
                                                   return_margins=True)
        ours = torch.stack([got[b, :, slots[b]] for b in range(batch)])[:, :, None]
        verdict = compare_codes(ours, want, d1, d2)
        assert verdict["clear_mismatches"] == 0 and verdict["agreement"] >= 0.999, verdict["agreement"]
    # the attention equals the plain decode over the updated cache, bit for bit,
    # and the oracle's decode of it within ATOL
    again = jkv.decode_attention(q.to(device), kc_got.to(device), vc_got.to(device), kt16, vt16, lens.to(device),
                                 window=window)
    assert torch.equal(out, again)
    for b, L in enumerate(lengths):
        e = _expect(q[b : b + 1], kc_got[b : b + 1], vc_got[b : b + 1], kt, vt, int(L), window, cap)
        err = float((out[b : b + 1].cpu().float() - e.float()).abs().max())
        assert err <= ATOL, f"row {b} length {L}: {err}"


def test_decode_append_entry_point_limits(device):
    # geometries the fused step does not serve are refused, not mis-served
    q, kc, vc, kt, vt = _case(3, 1, 8, 2, 32, 1, 4, 0, 512)
    knew = torch.zeros(1, 2, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="group dim 8"):
        jkv.decode_attention(q.to(device), kc.to(device), vc.to(device), kt.half().to(device), vt.half().to(device),
                             torch.tensor([5], dtype=torch.int32, device=device), window=512,
                             key_new=knew.to(device), value_new=knew.to(device))
    q, kc, vc, kt, vt = _case(3, 1, 8, 2, 16, 2, 8, 0, 512)
    with pytest.raises(ValueError, match="both"):
        jkv.decode_attention(q.to(device), kc.to(device), vc.to(device), kt.half().to(device), vt.half().to(device),
                             torch.tensor([5], dtype=torch.int32, device=device), window=512,
                             key_new=knew.to(device))


def test_attend_append_serving_loop(device):
    # PackedCodeCache.attend_append: each step's codes land in the ring slot
    # (the codec's greedy search, checked against the oracle), the output is
    # the plain decode over the updated cache bit for bit, and the cache
    # counts the token; the 4-slot ring wraps
    gen = torch.Generator().manual_seed(8621)
    batch, kvh, qh, cap = 3, 2, 8, 4
    kt = ref.synthetic_tables(gen, (kvh * 16, 2, 256, 8), (1.0, 0.5), stage_axis=1)
    vt = ref.synthetic_tables(gen, (kvh * 16, 2, 256, 8), (1.0, 0.5), stage_axis=1)
    kt16, vt16 = kt.half().to(device), vt.half().to(device)
    cache = jkv.PackedCodeCache(batch, kvh, 16, 2, capacity=cap, device=device)
    for step in range(6):
        k = ref.synthetic_states(gen, batch, kvh, 1)
        v = ref.synthetic_states(gen, batch, kvh, 1)
        q = torch.randn(batch, qh, 1, 128, generator=gen).half().to(device)
        out = cache.attend_append(q, k.to(device), v.to(device), kt16, vt16, window=cap)
        assert cache.length == step + 1 and torch.equal(cache.lengths.cpu(), torch.full((batch,), step + 1,
                                                                                          dtype=torch.int32))
        slot = step % cap
        for raw, tabs, got in ((k, kt, cache.key), (v, vt, cache.value)):
            _o, want, d1, d2 = ref.grouped_residual_vq(raw, tabs.reshape(kvh, 16, 2, 256, 8), prefixes=(2,),
                                                       return_margins=True)
            verdict = compare_codes(got[:, :, slot : slot + 1].cpu(), want, d1, d2)
            assert verdict["clear_mismatches"] == 0, f"step {step}"
        again = jkv.decode_attention(q, cache.key, cache.value, kt16, vt16, cache.lengths, window=cap,
                                     max_length=cache.length)
        assert torch.equal(out, again), f"step {step}"
        e = _expect(q.cpu(), cache.key.cpu(), cache.value.cpu(), kt, vt, step + 1, cap, cap)
        err = float((out.cpu().float() - e.float()).abs().max())
        assert err <= ATOL, f"step {step}: {err}"


def test_attend_append_refused_geometry_keeps_length(device):
    # a geometry the fused append does not serve (cq2: 32 groups of 4 dims)
    # raises before anything is written, and the cache still counts only the
    # tokens whose codes it holds
    gen = torch.Generator().manual_seed(8623)
    cache = jkv.PackedCodeCache(1, 2, 32, 1, capacity=16, device=device)
    codes = torch.randint(0, 256, (1, 2, 3, 32, 1), generator=gen, dtype=torch.uint8).to(device)
    cache.append(codes, codes)
    before_k, before_v = cache.key.clone(), cache.value.clone()
    t16 = ref.synthetic_tables(gen, (2 * 32, 1, 256, 4), (1.0,), stage_axis=1).half().to(device)
    q = torch.randn(1, 8, 1, 128, generator=gen).half().to(device)
    raw = ref.synthetic_states(gen, 1, 2, 1).to(device)
    with pytest.raises(ValueError):
        cache.attend_append(q, raw, raw, t16, t16, window=16)
    assert cache.length == 3 and torch.equal(cache.lengths.cpu(), torch.tensor([3], dtype=torch.int32))
    assert torch.equal(cache.key, before_k) and torch.equal(cache.value, before_v)
    # the fallback path then serves the step
    out = jkv.decode_attention(q, cache.key, cache.value, t16, t16, cache.lengths, window=16,
                               max_length=cache.length)
    assert out.shape == (1, 8, 1, 128)


def test_ragged_lengths_and_cache_append(device):
    batch = 3
    q, kc, vc, kt, vt = _case(5, batch, 8, 2, 16, 2, 8, 0, 1024)
    lengths = torch.tensor([1, 333, 1024], dtype=torch.int32)
    # capacity 1024 slots serves a 1024-token window
    out = jkv.decode_attention(q.to(device), kc.to(device), vc.to(device), kt.half().to(device),
                               vt.half().to(device), lengths.to(device), window=1024)
    # a 4096 window over sequences of at most 1024 tokens sees the same keys
    wide = jkv.decode_attention(q.to(device), kc.to(device), vc.to(device), kt.half().to(device),
                                vt.half().to(device), lengths.to(device), window=4096)
    assert torch.equal(wide, out)
    # but a declared length beyond the ring's capacity is refused
    with pytest.raises(ValueError, match="capacity"):
        jkv.decode_attention(q.to(device), kc.to(device), vc.to(device), kt.half().to(device),
                             vt.half().to(device), lengths.to(device), window=4096, max_length=2048)
    for b in range(batch):
        L = int(lengths[b])
        e = _expect(q[b : b + 1], kc[b : b + 1], vc[b : b + 1], kt, vt, L, 1024, 1024)
        err = float((out[b : b + 1].cpu().float() - e.float()).abs().max())
        assert err <= ATOL, f"batch {b} length {L}: {err}"
    # PackedCodeCache: appends land at position % capacity
    cache = jkv.PackedCodeCache(1, 2, 16, 2, capacity=8, device=device)
    seq = torch.randint(0, 256, (1, 2, 11, 16, 2), dtype=torch.uint8, device=device)
    cache.append(seq[:, :, :5], seq[:, :, :5])
    cache.append(seq[:, :, 5:11], seq[:, :, 5:11])
    assert cache.length == 11 and int(cache.lengths[0]) == 11
    for p in range(3, 11):
        assert torch.equal(cache.key[:, :, p % 8], seq[:, :, p])


def test_encode_append_matches_encode_then_append(device):
    # the codec's codes for one new token land in the ring slot in place
    gen = torch.Generator().manual_seed(8609)
    tables_k = ref.synthetic_tables(gen, (2 * 16, 2, 256, 8), (1.0, 0.5), stage_axis=1).to(device)
    tables_v = ref.synthetic_tables(gen, (2 * 16, 2, 256, 8), (1.0, 0.5), stage_axis=1).to(device)
    direct = jkv.PackedCodeCache(3, 2, 16, 2, capacity=4, device=device)
    fused = jkv.PackedCodeCache(3, 2, 16, 2, capacity=4, device=device)
    from jointkv_amd import _ops
    for _step in range(6):  # wraps the 4-slot ring
        k = ref.synthetic_states(gen, 3, 2, 1).to(device)
        v = ref.synthetic_states(gen, 3, 2, 1).to(device)
        _r, kc = _ops.rvq_encode(k, tables_k, groups=16, group_dim=8, exits=())
        _r, vc = _ops.rvq_encode(v, tables_v, groups=16, group_dim=8, exits=())
        direct.append(kc, vc)
        fused.encode_append(k, v, tables_k, tables_v, group_dim=8)
    assert torch.equal(direct.key, fused.key) and torch.equal(direct.value, fused.value)
    assert torch.equal(direct.lengths, fused.lengths) and fused.length == 6


def test_full_vector_cache_serving_loop(device):
    # R16-style codec (one 128-dim group, 16 stages): each step encodes the new
    # token into the ring slot and attends over the packed codes
    from jointkv_amd import _ops
    gen = torch.Generator().manual_seed(8611)
    stages, kvh, batch, cap = 16, 2, 2, 8
    sig = tuple(0.8 ** s for s in range(stages))
    tables_k = ref.synthetic_tables(gen, (kvh, stages, 256, 128), sig, stage_axis=1)
    tables_v = ref.synthetic_tables(gen, (kvh, stages, 256, 128), sig, stage_axis=1)
    tk, tv = tables_k.to(device), tables_v.to(device)
    direct = jkv.PackedCodeCache(batch, kvh, 1, stages, capacity=cap, device=device)
    fused = jkv.PackedCodeCache(batch, kvh, 1, stages, capacity=cap, device=device)
    for step in range(11):  # wraps the 8-slot ring
        k = ref.synthetic_states(gen, batch, kvh, 1).to(device)
        v = ref.synthetic_states(gen, batch, kvh, 1).to(device)
        _r, kc = _ops.rvq_encode(k, tk, groups=1, group_dim=128, exits=())
        _r, vc = _ops.rvq_encode(v, tv, groups=1, group_dim=128, exits=())
        direct.append(kc, vc)
        fused.encode_append(k, v, tk, tv, group_dim=128)
        print(f"full-vector serving step {step}", flush=True)
    assert torch.equal(direct.key, fused.key) and torch.equal(direct.value, fused.value)
    length = fused.length
    q = torch.randn(batch, 8, 1, 128, generator=gen).half()
    out = jkv.decode_attention(q.to(device), fused.key, fused.value, tk.half(), tv.half(), fused.lengths,
                               window=cap)
    expect = _expect(q, fused.key.cpu(), fused.value.cpu(), tables_k, tables_v, length, cap, cap)
    err = float((out.cpu().float() - expect.float()).abs().max())
    assert err <= ATOL, f"max abs error {err}"


@pytest.mark.parametrize("batch,qh,kvh,length,window,cap", [
    (2, 32, 8, 4096, 4096, 4096),   # config 4 heads, full window
    (1, 8, 2, 700, 256, 512),       # sliding window, ring wraps
    (3, 8, 8, 37, 4096, 64),        # short prefix, MHA
])
def test_decode_window_matches_oracle(device, batch, qh, kvh, length, window, cap):
    gen = torch.Generator().manual_seed(length + 7)
    q = torch.randn(batch, qh, 1, 128, generator=gen).half()
    kw = torch.randn(batch, kvh, cap, 128, generator=gen).half()
    vw = torch.randn(batch, kvh, cap, 128, generator=gen).half()
    print(f"window decode B={batch} QH={qh} KVH={kvh} len={length} win={window} cap={cap}", flush=True)
    out = jkv.decode_attention_window(
        q.to(device), kw.to(device), vw.to(device),
        torch.full((batch,), length, dtype=torch.int32, device=device), window=window)
    start = max(0, length - min(window, cap))
    pos = torch.arange(start, length)
    expect = ref.decode_attention(q, kw[:, :, pos % cap].contiguous(), vw[:, :, pos % cap].contiguous(),
                                  length - 1, pos)
    err = float((out.cpu().float() - expect.float()).abs().max())
    assert err <= ATOL, f"max abs error {err}"


def test_decoded_window_cache_equals_packed_decode(device):
    # the same codec step fills both caches; attention over the decoded window
    # and over the packed codes sees identical K̂/V̂ rows, so identical outputs
    gen = torch.Generator().manual_seed(8617)
    stages, kvh, batch, cap = 16, 2, 2, 8
    sig = tuple(0.8 ** s for s in range(stages))
    tk = ref.synthetic_tables(gen, (kvh, stages, 256, 128), sig, stage_axis=1).to(device)
    tv = ref.synthetic_tables(gen, (kvh, stages, 256, 128), sig, stage_axis=1).to(device)
    win = jkv.DecodedWindowCache(batch, kvh, 1, stages, capacity=cap, device=device)
    packed = jkv.PackedCodeCache(batch, kvh, 1, stages, capacity=cap, device=device)
    for step in range(11):  # wraps the 8-slot rings
        k = ref.synthetic_states(gen, batch, kvh, 1).to(device)
        v = ref.synthetic_states(gen, batch, kvh, 1).to(device)
        win.encode_append(k, v, tk, tv, group_dim=128)
        packed.encode_append(k, v, tk, tv, group_dim=128)
        q = torch.randn(batch, 8, 1, 128, generator=gen).half().to(device)
        a = win.attention(q)
        b = jkv.decode_attention(q, packed.key, packed.value, tk.half(), tv.half(), packed.lengths,
                                 window=cap, max_length=packed.length)
        assert torch.equal(a, b), f"step {step}: window and packed decode differ"
    assert torch.equal(win.codes.key, packed.key) and win.length == packed.length == 11
    assert win.payload_bytes() == packed.payload_bytes()


@pytest.mark.parametrize("stages", [16, 32])
def test_decoded_window_equals_packed_decode_over_many_splits(device, stages):
    # 700 tokens through 512-slot rings (the second append wraps), then
    # windows of 256, 512 and 300 tokens: every key tile and wave of both
    # kernels, ragged last tiles, GQA 4.  Within one split the two kernels
    # form the same products in the same order, so a window that each covers
    # with one split (256 tokens) gives the same bits; longer windows are
    # split at 512 tokens by the window kernel and at 256 by the packed one,
    # so their split combines add in different orders and the outputs agree
    # to fp32 rounding of the fp16 result
    from jointkv_amd import _ops

    gen = torch.Generator().manual_seed(8619 + stages)
    kvh, batch, cap = 2, 2, 512
    sig = tuple(0.8 ** s for s in range(stages))
    tk = ref.synthetic_tables(gen, (kvh, stages, 256, 128), sig, stage_axis=1).to(device)
    tv = ref.synthetic_tables(gen, (kvh, stages, 256, 128), sig, stage_axis=1).to(device)
    win = jkv.DecodedWindowCache(batch, kvh, 1, stages, capacity=cap, device=device)
    packed = jkv.PackedCodeCache(batch, kvh, 1, stages, capacity=cap, device=device)
    for tokens in (400, 300):
        k = ref.synthetic_states(gen, batch, kvh, tokens).to(device)
        v = ref.synthetic_states(gen, batch, kvh, tokens).to(device)
        (rk,), ck = _ops.rvq_encode(k, tk, groups=1, group_dim=128, exits=(stages,))
        (rv,), cv = _ops.rvq_encode(v, tv, groups=1, group_dim=128, exits=(stages,))
        win.append(ck, cv, rk, rv)
        packed.append(ck, cv)
    assert packed.length == 700
    q = torch.randn(batch, 8, 1, 128, generator=gen).half().to(device)
    for window in (256, cap, 300):
        print(f"window and packed decode S={stages} len=700 window={window}", flush=True)
        a = win.attention(q, window=window)
        b = jkv.decode_attention(q, packed.key, packed.value, tk.half(), tv.half(), packed.lengths,
                                 window=window, max_length=packed.length)
        if window <= 256:
            assert torch.equal(a, b), f"window {window}: window and packed decode differ"
        else:
            err = float((a.float() - b.float()).abs().max())
            assert err <= 2e-3 * max(1.0, float(a.float().abs().max())), f"window {window}: max abs difference {err}"
