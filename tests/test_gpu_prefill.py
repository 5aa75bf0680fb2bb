"""Prefill attention parity: HIP kernel vs the oracle's SDPA restatement."""

from __future__ import annotations

import pytest
import torch

import jointkv_amd as jkv
from jointkv_amd import _ops
from oracle import jointkv_oracle as ref

pytestmark = pytest.mark.gpu

ATOL = 2e-3  # max abs on attention outputs


def _case(seed, batch, qh, kvh, tokens, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, qh, tokens, 128, generator=gen).half()
    k = (torch.randn(batch, kvh, tokens, 128, generator=gen) * scale).half()
    v = torch.randn(batch, kvh, tokens, 128, generator=gen).half()
    return q, k, v


@pytest.mark.parametrize("batch,qh,kvh,tokens,starts,window", [
    (1, 32, 8, 200, (0,), 4096),          # Mistral GQA 4, window does not bind
    (2, 8, 2, 300, (0, 5000), 64),        # window binds, rotary at later positions
    (1, 4, 4, 130, (17,), 4096),          # MHA (one query head per kv head)
    (1, 16, 2, 100, (3,), 4096),          # GQA 8: two head groups per kv head
    (1, 4, 1, 1, (9,), 4096),             # one token sees only itself
])
def test_prefill_matches_oracle(device, batch, qh, kvh, tokens, starts, window):
    print(f"prefill B={batch} QH={qh} KVH={kvh} T={tokens} starts={starts} win={window}", flush=True)
    q, k, v = _case(101 + tokens, batch, qh, kvh, tokens)
    out = jkv.prefill_attention(q.to(device), k.to(device), v.to(device), list(starts), window=window)
    expect = ref.prefill_attention(q, k, v, starts, window=window)
    err = float((out.cpu().float() - expect.float()).abs().max())
    assert err <= ATOL, f"max abs error {err}"
    if tokens == 1:
        # softmax over one key: the output is that key's value row
        assert torch.equal(out.cpu()[0, :, 0], v[0, 0, 0].expand(qh, 128))


def test_prefill_from_codes_and_strided_inputs(device):
    # K/V as G2 codes rebuilt by the codec's decode, query as a strided view
    gen = torch.Generator().manual_seed(8601)
    tables = ref.synthetic_tables(gen, (8 * 16, 2, 256, 8), (1.0, 0.5), stage_axis=1)
    t16 = tables.half()
    kc = torch.randint(0, 256, (1, 8, 256, 16, 2), generator=gen, dtype=torch.uint8)
    vc = torch.randint(0, 256, (1, 8, 256, 16, 2), generator=gen, dtype=torch.uint8)
    big = torch.randn(1, 256, 32, 128, generator=gen).half()  # [B,T,QH,D] as a projection lays it out
    q = big.transpose(1, 2)
    khat = ref.frozen_decode(kc, t16.float(), 2, torch.float16)
    vhat = ref.frozen_decode(vc, (t16 * 0.5).float(), 2, torch.float16)
    expect = ref.prefill_attention(q.contiguous(), khat, vhat, (40,))
    outs = [jkv.prefill_attention_from_codes(q.to(device), kc.to(device), vc.to(device), t16.to(device),
                                             (t16 * 0.5).to(device), 40, fused=fused) for fused in (False, True)]
    assert torch.equal(outs[0], outs[1])
    err = float((outs[0].cpu().float() - expect.float()).abs().max())
    assert err <= ATOL, f"max abs error {err}"


def _decoded_then_attended(q, kc, vc, kt16, vt16, starts, window, device):
    """The two-launch path: jkv_rvq_decode of K̂ and V̂, then the prefill."""

    stages = int(kc.shape[-1])
    khat = _ops.rvq_decode(kc, kt16.float(), depth=stages, dtype=torch.float16)
    vhat = _ops.rvq_decode(vc, vt16.float(), depth=stages, dtype=torch.float16)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=device)
    top = int(max(starts)) + int(q.shape[2]) - 1
    st = torch.tensor(starts, dtype=torch.int32, device=device)
    out = _ops.prefill_attention(q, khat, vhat, st, window=window, rope_theta=10000.0, max_position=top, lse=lse)
    return out, lse, khat, vhat


@pytest.mark.parametrize("batch,qh,kvh,tokens,stages,starts,window,cap", [
    (1, 32, 8, 256, 2, (0,), 4096, None),          # Mistral heads, GSRQ-2
    (2, 8, 2, 300, 2, (0, 5000), 64, None),        # window binds, ragged last tile, later positions
    (1, 8, 2, 200, 1, (7,), 4096, None),           # one stage
    (2, 16, 2, 97, 2, (3, 11), 40, 160),           # GQA 8; codes as a slice of a longer code cache
    (1, 4, 1, 1, 2, (9,), 4096, None),             # one token
    (1, 32, 8, 2048, 2, (0,), 4096, None),         # config 4 prefill chunk, one batch row
])
def test_prefill_codes_fused_equals_decode_then_attend(device, batch, qh, kvh, tokens, stages, starts, window,
                                                        cap):
    # the fused kernel rebuilds K̂/V̂ in registers with the codec's own
    # arithmetic, so its output and lse carry the two-launch path's bits
    print(f"prefill codes B={batch} QH={qh} KVH={kvh} T={tokens} S={stages} starts={starts} win={window} "
          f"cap={cap}", flush=True)
    gen = torch.Generator().manual_seed(9100 + tokens)
    tables = ref.synthetic_tables(gen, (kvh * 16, stages, 256, 8), (1.0, 0.5)[:stages], stage_axis=1)
    kt16, vt16 = tables.half().to(device), (tables * 0.7).half().to(device)
    rows = cap or tokens
    kc = torch.randint(0, 256, (batch, kvh, rows, 16, stages), generator=gen, dtype=torch.uint8).to(device)
    vc = torch.randint(0, 256, (batch, kvh, rows, 16, stages), generator=gen, dtype=torch.uint8).to(device)
    kc, vc = kc[:, :, :tokens], vc[:, :, :tokens]
    q = torch.randn(batch, qh, tokens, 128, generator=gen).half().to(device)
    want, want_lse, khat, vhat = _decoded_then_attended(q, kc, vc, kt16, vt16, starts, window, device)
    lse = torch.empty_like(want_lse)
    st = torch.tensor(starts, dtype=torch.int32, device=device)
    top = int(max(starts)) + tokens - 1
    got = _ops.prefill_attention_codes(q, kc, vc, kt16, vt16, st, window=window, rope_theta=10000.0,
                                       max_position=top, lse=lse)
    assert torch.equal(got, want), float((got.float() - want.float()).abs().max())
    assert torch.equal(lse, want_lse)
    if tokens <= 300:
        # and the oracle on the codec's reconstruction
        expect = ref.prefill_attention(q.cpu(), khat.cpu(), vhat.cpu(), starts, window=window)
        err = float((got.cpu().float() - expect.float()).abs().max())
        assert err <= ATOL, f"max abs error {err}"


def test_prefill_codes_other_geometry_decodes_first(device):
    # 8 groups of 16 dims lie outside the fused kernel: the API decodes K̂/V̂
    # and attends, with the same result as the oracle, and refuses fused=True
    gen = torch.Generator().manual_seed(515)
    tables = ref.synthetic_tables(gen, (2 * 8, 2, 64, 16), (1.0, 0.5), stage_axis=1)
    t16 = tables.half()
    kc = torch.randint(0, 64, (1, 2, 90, 8, 2), generator=gen, dtype=torch.uint8)
    vc = torch.randint(0, 64, (1, 2, 90, 8, 2), generator=gen, dtype=torch.uint8)
    q = torch.randn(1, 8, 90, 128, generator=gen).half()
    assert not _ops.prefill_codes_supported(kc, t16)
    with pytest.raises(ValueError, match="fused prefill"):
        jkv.prefill_attention_from_codes(q.to(device), kc.to(device), vc.to(device), t16.to(device),
                                         t16.to(device), 5, fused=True)
    out = jkv.prefill_attention_from_codes(q.to(device), kc.to(device), vc.to(device), t16.to(device),
                                           t16.to(device), 5)
    khat = ref.frozen_decode(kc, t16.float(), 2, torch.float16)
    vhat = ref.frozen_decode(vc, t16.float(), 2, torch.float16)
    expect = ref.prefill_attention(q, khat, vhat, (5,))
    assert float((out.cpu().float() - expect.float()).abs().max()) <= ATOL


def test_prefill_codes_rejects_bad_geometry(device):
    gen = torch.Generator().manual_seed(3)
    t16 = ref.synthetic_tables(gen, (16, 2, 256, 8), (1.0, 0.5), stage_axis=1).half().to(device)
    kc = torch.randint(0, 256, (1, 1, 8, 16, 2), generator=gen, dtype=torch.uint8).to(device)
    q = torch.randn(1, 4, 8, 128, generator=gen).half().to(device)
    st = torch.zeros(1, dtype=torch.int32, device=device)
    kw = dict(window=4096, rope_theta=10000.0, max_position=7)
    with pytest.raises(ValueError):  # key and value codes differ
        _ops.prefill_attention_codes(q, kc, kc[:, :, :4], t16, t16, st, **kw)
    with pytest.raises(ValueError):  # tables for two kv heads
        _ops.prefill_attention_codes(q, kc, kc, torch.cat([t16, t16]), torch.cat([t16, t16]), st, **kw)
    with pytest.raises(ValueError):  # query rows differ from the code rows
        _ops.prefill_attention_codes(q[:, :, :5], kc, kc, t16, t16, st, **kw)


def test_prefill_config4_chunk_one_row(device):
    # config 4 prefill chunk (2048 tokens, 32/8 heads) for one batch row
    q, k, v = _case(8601, 1, 32, 8, 2048)
    out = jkv.prefill_attention(q.to(device), k.to(device), v.to(device), 0)
    expect = ref.prefill_attention(q, k, v, (0,))
    err = float((out.cpu().float() - expect.float()).abs().max())
    assert err <= ATOL, f"max abs error {err}"


def test_prefill_batch16_block_mapping(device):
    # the benchmarked batch of 16 (32/8 heads): every batch row at a 256-token
    # chunk against the oracle, then rows 0, 9 and 15 of the full 2048-token
    # config-4 chunk, so the block -> (batch, kv head, head group, rows)
    # mapping of the launch the bench times is checked at its own grid
    q, k, v = _case(8602, 16, 32, 8, 256)
    out = jkv.prefill_attention(q.to(device), k.to(device), v.to(device), 0)
    expect = ref.prefill_attention(q, k, v, (0,) * 16)
    err = float((out.cpu().float() - expect.float()).abs().max())
    assert err <= ATOL, f"T=256 max abs error {err}"
    q, k, v = _case(8603, 16, 32, 8, 2048)
    out = jkv.prefill_attention(q.to(device), k.to(device), v.to(device), 0).cpu()
    for b in (0, 9, 15):
        print(f"prefill B=16 T=2048 row {b}", flush=True)
        expect = ref.prefill_attention(q[b : b + 1], k[b : b + 1], v[b : b + 1], (0,))
        err = float((out[b : b + 1].float() - expect.float()).abs().max())
        assert err <= ATOL, f"T=2048 row {b}: max abs error {err}"


def test_prefill_rejects_bad_geometry(device):
    q, k, v = _case(1, 1, 4, 2, 8)
    with pytest.raises(ValueError):
        jkv.prefill_attention(q[..., :64].contiguous().to(device), k.to(device), v.to(device), 0)
    with pytest.raises(ValueError):
        jkv.prefill_attention(q.to(device), k.to(device), v[:, :, :4].to(device), 0)
