"""Prefill attention parity: HIP kernel vs the oracle's SDPA restatement."""

from __future__ import annotations

import pytest
import torch

import jointkv_amd as jkv
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
    out = jkv.prefill_attention_from_codes(q.to(device), kc.to(device), vc.to(device), t16.to(device),
                                           (t16 * 0.5).to(device), 40)
    khat = ref.frozen_decode(kc, t16.float(), 2, torch.float16)
    vhat = ref.frozen_decode(vc, (t16 * 0.5).float(), 2, torch.float16)
    expect = ref.prefill_attention(q.contiguous(), khat, vhat, (40,))
    err = float((out.cpu().float() - expect.float()).abs().max())
    assert err <= ATOL, f"max abs error {err}"


def test_prefill_config4_chunk_one_row(device):
    # config 4 prefill chunk (2048 tokens, 32/8 heads) for one batch row
    q, k, v = _case(8601, 1, 32, 8, 2048)
    out = jkv.prefill_attention(q.to(device), k.to(device), v.to(device), 0)
    expect = ref.prefill_attention(q, k, v, (0,))
    err = float((out.cpu().float() - expect.float()).abs().max())
    assert err <= ATOL, f"max abs error {err}"


def test_prefill_rejects_bad_geometry(device):
    q, k, v = _case(1, 1, 4, 2, 8)
    with pytest.raises(ValueError):
        jkv.prefill_attention(q[..., :64].contiguous().to(device), k.to(device), v.to(device), 0)
    with pytest.raises(ValueError):
        jkv.prefill_attention(q.to(device), k.to(device), v[:, :, :4].to(device), 0)
