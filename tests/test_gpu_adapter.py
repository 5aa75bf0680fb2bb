"""Closed-loop attention adapter on the MI355X: the prefill row normaliser,
its HIP value gradient, and one layer's V-only step against the oracle."""

from __future__ import annotations

import pytest
import torch

import jointkv_amd as jkv
from jointkv_amd import _ops
from jointkv_amd.attention import _start_tensor
from jointkv_amd.closed_loop_attention import AttentionWeights, closed_loop_attention
from oracle import jointkv_oracle as ref

pytestmark = pytest.mark.gpu

LSE_ATOL = 2e-3      # natural-log row normaliser, fp32 math on fp16 operands
DV_RTOL = 3e-3       # dV̂ against fp32 autograd: P enters the MFMA as fp16 (2^-11)
STEP_RTOL = 1e-2     # table gradients after fp16 projections, fp16 dO and fp16 dV̂


def _case(seed, batch, qh, kvh, tokens):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, qh, tokens, 128, generator=gen).half()
    k = torch.randn(batch, kvh, tokens, 128, generator=gen).half()
    v = torch.randn(batch, kvh, tokens, 128, generator=gen).half()
    d = torch.randn(batch, qh, tokens, 128, generator=gen).half()
    return q, k, v, d


@pytest.mark.parametrize("batch,qh,kvh,tokens,starts,window", [
    (1, 32, 8, 200, (0,), 4096),        # Mistral GQA 4, window does not bind
    (2, 8, 2, 301, (0, 5000), 64),      # window binds; ragged key blocks and row tiles
    (1, 4, 4, 70, (17,), 4096),         # one query head per kv head
    (1, 4, 2, 45, (3,), 4096),          # GQA 2
    (1, 16, 2, 96, (0,), 4096),         # GQA 8
    (1, 4, 1, 1, (9,), 4096),           # one token
    (1, 8, 2, 600, (0,), 4096),         # key blocks' rows split in two runs (workspace + reduce)
    (1, 8, 2, 1030, (40,), 4096),       # three runs, ragged last tile
    (1, 8, 2, 1500, (0,), 256),         # window binds over many tiles: blocks meet chunks that wrap the slots
])
def test_lse_and_value_grad_match_oracle(device, batch, qh, kvh, tokens, starts, window):
    ws = int(_ops._lib.load().jkv_prefill_value_grad_workspace_bytes(batch, qh, kvh, tokens, window))
    print(f"value grad B={batch} QH={qh} KVH={kvh} T={tokens} starts={starts} win={window} ws={ws}", flush=True)
    q, k, v, d = _case(900 + tokens, batch, qh, kvh, tokens)
    qd, kd, vd, dd = (t.to(device) for t in (q, k, v, d))
    st, top = _start_tensor(list(starts), batch, tokens, qd.device)
    lse = torch.empty(batch, qh, tokens, dtype=torch.float32, device=device)
    out = _ops.prefill_attention(qd, kd, vd, st, window=window, rope_theta=10000.0, max_position=top, lse=lse)
    # the forward is unchanged by asking for lse
    assert torch.equal(out, jkv.prefill_attention(qd, kd, vd, list(starts), window=window))
    lse_ref = ref.prefill_lse(q, k, starts, window=window)
    err = float((lse.cpu() - lse_ref).abs().max())
    assert err <= LSE_ATOL, f"lse max abs error {err}"
    dv = _ops.prefill_attention_value_grad(qd, kd, dd, lse, st, window=window, rope_theta=10000.0,
                                           max_position=top)
    dv_ref = ref.prefill_value_grad(q, k, v, d, starts, window=window)
    scale = float(dv_ref.abs().max())
    err = float((dv.cpu() - dv_ref).abs().max())
    print(f"  lse err {float((lse.cpu() - lse_ref).abs().max()):.2e}  dV err {err:.2e} of {scale:.2e}", flush=True)
    assert err <= DV_RTOL * scale, f"dV max abs error {err} (scale {scale})"
    # deterministic: a second call gives the same bits
    again = _ops.prefill_attention_value_grad(qd, kd, dd, lse, st, window=window, rope_theta=10000.0,
                                              max_position=top)
    assert torch.equal(dv, again)


def test_autograd_value_path(device):
    q, k, v, d = _case(31, 1, 8, 2, 64)
    qd, kd, dd = q.to(device), k.to(device), d.to(device)
    vd = v.to(device).requires_grad_(True)
    out = jkv.prefill_attention(qd, kd, vd, 0, window=4096)
    out.backward(dd)
    assert vd.grad.dtype == torch.float16
    dv_ref = ref.prefill_value_grad(q, k, v, d, (0,), window=4096)
    assert float((vd.grad.cpu().float() - dv_ref).abs().max()) <= DV_RTOL * float(dv_ref.abs().max())


@pytest.mark.parametrize("batch,qh,kvh,tokens,starts,window", [
    (1, 32, 8, 200, (0,), 4096),        # Mistral GQA 4
    (2, 8, 2, 301, (0, 5000), 64),      # window binds, later positions, ragged tiles
    (1, 4, 4, 70, (17,), 4096),         # one query head per kv head
    (1, 4, 2, 45, (3,), 4096),          # GQA 2
    (1, 16, 2, 96, (0,), 4096),         # GQA 8: two head groups per kv head
    (1, 8, 2, 600, (0,), 4096),         # rows and keys split in runs (workspace + reduce)
    (1, 8, 2, 1500, (0,), 256),         # window binds over many tiles: chunks wrap the slots
    (1, 4, 1, 1, (9,), 4096),           # one token: one step in every walk
    (2, 8, 2, 33, (0, 31), 16),         # one row past a tile, window of 16
])
def test_full_backward_matches_oracle(device, batch, qh, kvh, tokens, starts, window):
    print(f"backward B={batch} QH={qh} KVH={kvh} T={tokens} starts={starts} win={window}", flush=True)
    q, k, v, d = _case(1900 + tokens, batch, qh, kvh, tokens)
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    out = jkv.prefill_attention(qd, kd, vd, list(starts), window=window)
    out.backward(d.to(device))
    dq_ref, dk_ref = ref.prefill_qk_grad(q, k, v, d, starts, window=window)
    dv_ref = ref.prefill_value_grad(q, k, v, d, starts, window=window)
    for name, got, want in (("dq", qd.grad, dq_ref), ("dk", kd.grad, dk_ref), ("dv", vd.grad, dv_ref)):
        assert got.dtype == torch.float16
        scale = float(want.abs().max())
        err = float((got.cpu().float() - want).abs().max())
        print(f"  {name} err {err:.2e} of {scale:.2e}", flush=True)
        assert err <= DV_RTOL * scale + 1e-3, f"{name} max abs error {err} (scale {scale})"


@pytest.mark.parametrize("batch,qh,kvh,tokens,starts,window", [
    (1, 32, 8, 200, (0,), 4096),        # Mistral GQA 4
    (2, 8, 2, 301, (0, 5000), 64),      # window binds, later positions, ragged tiles
    (1, 8, 2, 600, (0,), 4096),         # keys split in runs (workspace + reduce)
])
def test_key_grad_entry_matches_backward_key_leg(device, batch, qh, kvh, tokens, starts, window):
    # jkv_prefill_attention_key_grad given delta = rowsum(dO * O) from the
    # host equals the full backward's key leg (which forms delta itself)
    from jointkv_amd import _lib

    print(f"key grad B={batch} QH={qh} KVH={kvh} T={tokens} starts={starts} win={window}", flush=True)
    q, k, v, d = _case(2300 + tokens, batch, qh, kvh, tokens)
    qd, kd, vd, dd = (t.to(device) for t in (q, k, v, d))
    st = torch.tensor(starts, dtype=torch.int32, device=device)
    max_pos = max(starts) + tokens - 1
    lse = torch.empty(batch, qh, tokens, dtype=torch.float32, device=device)
    out = _ops.prefill_attention(qd, kd, vd, st, window=window, rope_theta=10000.0, max_position=max_pos, lse=lse)
    _dq, dk_full, _dv = _ops.prefill_attention_backward(
        qd, kd, vd, out, dd, lse, st, window=window, rope_theta=10000.0, max_position=max_pos,
        need=(False, True, False))
    delta = (dd.float() * out.float()).sum(-1).contiguous()
    table = _ops.rope_table(device, 10000.0, max_pos + 1)
    lib = _lib.load()
    ws = int(lib.jkv_prefill_value_grad_workspace_bytes(batch, qh, kvh, tokens, window))
    work = torch.empty(max(ws, 1), dtype=torch.uint8, device=device)
    dk = torch.empty(batch, kvh, tokens, 128, dtype=torch.float32, device=device)
    _lib.check(lib.jkv_prefill_attention_key_grad(
        qd.data_ptr(), *qd.stride()[:3], kd.data_ptr(), *kd.stride()[:3], vd.data_ptr(), *vd.stride()[:3],
        dd.data_ptr(), *dd.stride()[:3], lse.data_ptr(), delta.data_ptr(), batch, qh, kvh, tokens, 128,
        st.data_ptr(), window, table.data_ptr(), int(table.shape[0]), dk.data_ptr(), work.data_ptr(), ws,
        _lib.stream_handle(device)))
    scale = float(dk_full.abs().max())
    err = float((dk - dk_full).abs().max())
    print(f"  dk err {err:.2e} of {scale:.2e}", flush=True)
    # the two deltas are fp32 sums of the same fp16 products in different orders
    assert err <= 1e-4 * scale + 1e-6


@pytest.mark.parametrize("batch,qh,kvh,tokens,starts,window", [
    (2, 8, 2, 300, (0, 40), 4096),      # GQA 4, ragged tiles, two start positions
    (1, 32, 8, 200, (0,), 64),          # Mistral heads, window binds
])
def test_strided_layouts_equal_contiguous(device, batch, qh, kvh, tokens, starts, window):
    # q, K, V and dO as [B,T,H,D] tensors viewed as [B,H,T,D] (the layout a
    # projection leaves): the forward, the value gradient and the full
    # backward address them by their strides and must give the same bits as
    # on contiguous copies
    print(f"strided B={batch} QH={qh} KVH={kvh} T={tokens} starts={starts} win={window}", flush=True)
    gen = torch.Generator().manual_seed(4400 + tokens)
    views = [torch.randn(batch, tokens, h, 128, generator=gen).half().to(device).transpose(1, 2)
             for h in (qh, kvh, kvh, qh)]
    q, k, v, d = views
    assert not q.is_contiguous() and q.stride(2) == qh * 128
    qc, kc, vc, dc = (t.contiguous() for t in views)
    st = torch.tensor(starts, dtype=torch.int32, device=device)
    max_pos = max(starts) + tokens - 1
    kw = dict(window=window, rope_theta=10000.0, max_position=max_pos)
    lse_s = torch.empty(batch, qh, tokens, dtype=torch.float32, device=device)
    lse_c = torch.empty_like(lse_s)
    out_s = _ops.prefill_attention(q, k, v, st, lse=lse_s, **kw)
    out_c = _ops.prefill_attention(qc, kc, vc, st, lse=lse_c, **kw)
    assert torch.equal(out_s, out_c) and torch.equal(lse_s, lse_c)
    dv_s = _ops.prefill_attention_value_grad(q, k, d, lse_c, st, **kw)
    dv_c = _ops.prefill_attention_value_grad(qc, kc, dc, lse_c, st, **kw)
    assert torch.equal(dv_s, dv_c)
    grads_s = _ops.prefill_attention_backward(q, k, v, out_c, d, lse_c, st, **kw)
    grads_c = _ops.prefill_attention_backward(qc, kc, vc, out_c, dc, lse_c, st, **kw)
    for name, a, b in zip(("dq", "dk", "dv"), grads_s, grads_c):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("tokens,stages,whitened", [(96, 2, False), (150, 4, True)])
def test_closed_loop_attention_value_step(device, tokens, stages, whitened):
    # a small decoder layer (4 query heads, 1 kv head, head_dim 128) with
    # full-vector codebooks; synthetic hidden states and upstream gradient
    print(f"adapter step T={tokens} S={stages} whitened={whitened}", flush=True)
    gen = torch.Generator().manual_seed(77 + tokens)
    hidden_size, kvh = 512, 1
    hidden = (torch.randn(1, tokens, hidden_size, generator=gen) * 0.5).half()
    w = {name: (torch.randn(rows, hidden_size, generator=gen) / hidden_size ** 0.5).half()
         for name, rows in (("q", hidden_size), ("k", 128 * kvh), ("v", 128 * kvh), ("o", hidden_size))}
    sig = tuple(0.8 ** s for s in range(stages))
    ktab = ref.synthetic_tables(gen, (kvh, stages, 256, 128), sig, stage_axis=1) * 0.5
    vtab = ref.synthetic_tables(gen, (kvh, stages, 256, 128), sig, stage_axis=1) * 0.5
    whitener = (torch.triu(torch.randn(kvh, 128, 128, generator=gen) * 0.05) + torch.eye(128)) if whitened else None
    d_proj = (torch.randn(1, tokens, hidden_size, generator=gen) * 0.1).half()

    codec = jkv.ClosedLoopUniformResidualVQ([ktab], [vtab], [whitener], depth=stages, dynamic_bpa=1.0).to(device)
    weights = AttentionWeights(*(w[n].to(device) for n in ("q", "k", "v", "o")))
    projected, traj = closed_loop_attention(hidden.to(device), weights, codec, 0, trajectory_epsilon=1e-8)
    projected.backward(d_proj.to(device))
    grad = codec.value_tables[0].grad

    expect_out, expect_grad = ref.closed_loop_attention_value_step(hidden, w, ktab, vtab, d_proj, depth=stages,
                                                                   key_whitener=whitener)
    out_err = float((projected.detach().cpu().float() - expect_out.float()).abs().max())
    assert out_err <= 2e-3 + 2e-3 * float(expect_out.abs().max()), f"projected max abs error {out_err}"
    rel = float((grad.cpu() - expect_grad).norm() / expect_grad.norm())
    print(f"  projected err {out_err:.2e}  table-grad relative error {rel:.2e}", flush=True)
    assert rel <= STEP_RTOL, f"value-table gradient relative error {rel}"
    traj = float(traj.detach())
    assert traj >= 0.0 and traj == traj
    # the frozen K tables take no gradient
    assert codec.key_tables[0].grad is None


def test_closed_loop_attention_hidden_gradient(device):
    # hidden states that require grad: the attention's query and key legs
    # carry dL/d hidden down (as to a lower layer in the 32-layer trajectory)
    gen = torch.Generator().manual_seed(515)
    tokens, stages, hidden_size, kvh = 80, 2, 512, 1
    hidden = (torch.randn(1, tokens, hidden_size, generator=gen) * 0.5).half()
    w = {name: (torch.randn(rows, hidden_size, generator=gen) / hidden_size ** 0.5).half()
         for name, rows in (("q", hidden_size), ("k", 128 * kvh), ("v", 128 * kvh), ("o", hidden_size))}
    sig = tuple(0.8 ** s for s in range(stages))
    ktab = ref.synthetic_tables(gen, (kvh, stages, 256, 128), sig, stage_axis=1) * 0.5
    vtab = ref.synthetic_tables(gen, (kvh, stages, 256, 128), sig, stage_axis=1) * 0.5
    d_proj = (torch.randn(1, tokens, hidden_size, generator=gen) * 0.1).half()
    codec = jkv.ClosedLoopUniformResidualVQ([ktab], [vtab], [None], depth=stages, dynamic_bpa=1.0).to(device)
    weights = AttentionWeights(*(w[n].to(device) for n in ("q", "k", "v", "o")))
    hd = hidden.to(device).requires_grad_(True)
    projected = closed_loop_attention(hd, weights, codec, 0)
    projected.backward(d_proj.to(device))
    _out, expect_grad, expect_hidden = ref.closed_loop_attention_value_step(
        hidden, w, ktab, vtab, d_proj, depth=stages, hidden_grad=True)
    rel_t = float((codec.value_tables[0].grad.cpu() - expect_grad).norm() / expect_grad.norm())
    rel_h = float((hd.grad.cpu().float() - expect_hidden).norm() / expect_hidden.norm())
    print(f"  table-grad relative error {rel_t:.2e}  hidden-grad relative error {rel_h:.2e}", flush=True)
    assert rel_t <= STEP_RTOL and rel_h <= STEP_RTOL
