"""Pins of the CPU oracle (no GPU): brute force, closed forms, known answers.

Each test is chosen so that a plausible mistake in the oracle (a dropped
norm term, a wrong sign, a transposed operand, a missing fp16 deploy round
trip, a stage-order slip) fails it.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import bruteforce as bf
from oracle import jointkv_oracle as ref
from parity import assert_codes_with_exact_floor, bruteforce_rvq_codes, compare_codes


def _clear(d1: np.ndarray, d2: np.ndarray, margin: float) -> np.ndarray:
    return (d2 - d1) > margin * np.maximum(d1, 1e-30)


def _assert_margins_track(d1, d2, bd1, bd2, rows):
    """The oracle's fp32 best and second-best distances equal the float64
    brute force's on the given rows (where the codes up to this stage match):
    the second-best distance decides which codes must be bit-exact, so a slip
    in it (e.g. the best distance returned twice) must not go unseen."""

    d1, d2 = np.asarray(d1, dtype=np.float64), np.asarray(d2, dtype=np.float64)
    np.testing.assert_allclose(d1[rows], bd1[rows], rtol=1e-3, atol=1e-4)
    np.testing.assert_allclose(d2[rows], bd2[rows], rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("seed,dim,clusters", [(1, 3, 4), (2, 4, 16), (3, 8, 256), (4, 4, 256)])
def test_nearest_search_matches_fp64_bruteforce(seed, dim, clusters):
    gen = torch.Generator().manual_seed(seed)
    states = torch.randn(2, 300, dim, generator=gen)
    table = torch.randn(2, clusters, dim, generator=gen)
    idx = ref.nearest_indices(states, table, token_chunk_size=37)
    for h in range(2):
        codes, d1, d2 = bf.rvq_encode(states[h].double().numpy(), table[h][None].double().numpy())
        clear = _clear(d1[:, 0], d2[:, 0], 1e-5)
        assert clear.mean() > 0.9
        assert np.array_equal(idx[h].numpy()[clear], codes[clear, 0])


def test_residual_stages_match_fp64_bruteforce_hierarchically():
    gen = torch.Generator().manual_seed(11)
    states = ref.synthetic_states(gen, 1, 2, 200, 8, outliers=1)
    tables = ref.synthetic_tables(gen, (2, 3, 64, 8), (1.0, 0.5, 0.25), stage_axis=1)
    _out, codes, d1, d2 = ref.hard_residual_vq_exits(states, tables, prefixes=(3,), return_margins=True)
    for h in range(2):
        bcodes, bd1, bd2 = bf.rvq_encode(states[0, h].double().numpy(), tables[h].double().numpy())
        ours = codes[0, h].numpy().astype(np.int32)
        matched = np.ones(ours.shape[0], dtype=bool)
        for s in range(3):
            clear = _clear(bd1[:, s], bd2[:, s], 1e-5) & matched
            assert np.array_equal(ours[clear, s], bcodes[clear, s])
            # best and second-best distances of stage s, where stages < s matched
            _assert_margins_track(d1[0, h, :, s].numpy(), d2[0, h, :, s].numpy(), bd1[:, s], bd2[:, s], matched)
            matched &= ours[:, s] == bcodes[:, s]
        assert matched.mean() > 0.98


def test_margin_pin_catches_a_second_best_slip():
    # plant the slip in the oracle's output: the best distance returned as the
    # second best (vals[..., 0] for vals[..., 1]) must fail the pin
    gen = torch.Generator().manual_seed(12)
    states = ref.synthetic_states(gen, 1, 1, 150, 8, outliers=1)
    tables = ref.synthetic_tables(gen, (1, 2, 64, 8), (1.0, 0.5), stage_axis=1)
    _out, codes, d1, d2 = ref.hard_residual_vq_exits(states, tables, prefixes=(2,), return_margins=True)
    bcodes, bd1, bd2 = bf.rvq_encode(states[0, 0].double().numpy(), tables[0].double().numpy())
    rows = codes[0, 0, :, 0].numpy() == bcodes[:, 0]
    _assert_margins_track(d1[0, 0, :, 0].numpy(), d2[0, 0, :, 0].numpy(), bd1[:, 0], bd2[:, 0], rows)
    with pytest.raises(AssertionError):
        _assert_margins_track(d1[0, 0, :, 0].numpy(), d1[0, 0, :, 0].numpy(), bd1[:, 0], bd2[:, 0], rows)
    # and the clear-margin rule then judges no code at all: the check it feeds
    # would be switched off
    assert compare_codes(codes, codes, d1, d1)["clear_mismatches"] == 0


def test_exits_equal_decode_of_codes_and_fp16_codewords():
    # Relation of closed_loop_vq exits and the literal fp16-deployed decode
    # (tests/test_closed_loop_vq.py:54-99 in the reference): a master value
    # that does not survive fp16 must not change codes or reconstruction.
    gen = torch.Generator().manual_seed(10)
    states = torch.randn(1, 2, 9, 4, generator=gen, dtype=torch.float32).half()
    tables = torch.randn(2, 3, 4, 4, generator=gen) + 1.234567e-4
    out, codes = ref.hard_residual_vq_exits(states, tables, prefixes=(1, 2, 3), token_chunk_size=4)
    out16, codes16 = ref.hard_residual_vq_exits(states, tables.half().float(), prefixes=(1, 2, 3))
    assert torch.equal(codes, codes16)
    for depth in (1, 2, 3):
        assert torch.equal(out[depth].detach(), out16[depth].detach())
        decoded = ref.frozen_decode(codes.unsqueeze(3), tables, depth, torch.float16)
        assert torch.equal(out[depth].detach(), decoded)


def test_frozen_decode_of_grouped_codes_equals_the_grouped_exits():
    # the deployment layout [B,H,T,G,S] codes with [H*G,S,K,d] tables at G = 16
    # groups of 8 dims: decoding the grouped operator's codes rebuilds its exits
    # bit for bit at every depth (a group or stage axis taken in the wrong order
    # lands codewords in the wrong 8-dim slice)
    gen = torch.Generator().manual_seed(16)
    states = ref.synthetic_states(gen, 2, 2, 24)
    tables = ref.synthetic_tables(gen, (2, 16, 2, 256, 8), (1.0, 0.5), stage_axis=2)
    exits, codes = ref.grouped_residual_vq(states, tables, prefixes=(1, 2))
    assert codes.shape == (2, 2, 24, 16, 2)
    for depth in (1, 2):
        got = ref.frozen_decode(codes, tables.reshape(32, 2, 256, 8), depth, torch.float16)
        assert torch.equal(got, exits[depth].detach())


def test_chunk_size_does_not_change_codes():
    gen = torch.Generator().manual_seed(7)
    states = torch.randn(1, 2, 12, 4, generator=gen)
    tables = torch.randn(2, 3, 4, 4, generator=gen)
    _a, ca = ref.hard_residual_vq_exits(states, tables, prefixes=(3,), token_chunk_size=5)
    _b, cb = ref.hard_residual_vq_exits(states, tables, prefixes=(3,), token_chunk_size=1024)
    assert torch.equal(ca, cb)


def test_hard_gradient_known_answer_one_dimensional():
    # tests/test_closed_loop_vq.py:131-162: state 0.1, words [0,1,10,20]:
    # the hard backward puts exactly 1.0 on word 0 and nothing elsewhere.
    states = torch.tensor([[[[0.1]]]], requires_grad=True)
    tables = torch.tensor([[[[0.0], [1.0], [10.0], [20.0]]]], requires_grad=True)
    out, codes = ref.hard_residual_vq_exits(states, tables, prefixes=(1,), straight_through_states=False)
    out[1].sum().backward()
    assert int(codes.item()) == 0
    assert tables.grad[0, 0, 0].item() == 1.0
    assert tables.grad[0, 0, 1:].count_nonzero() == 0
    assert states.grad is None or states.grad.count_nonzero() == 0


def test_autograd_gradient_equals_closed_form_and_bruteforce():
    gen = torch.Generator().manual_seed(43)
    states = torch.randn(2, 2, 40, 8, generator=gen).requires_grad_()
    tables = torch.randn(2, 3, 16, 8, generator=gen).requires_grad_()
    out, codes = ref.hard_residual_vq_exits(states, tables, prefixes=(2, 3))
    g2 = torch.randn(out[2].shape, generator=gen)
    g3 = torch.randn(out[3].shape, generator=gen)
    (out[2] * g2 + out[3] * g3).sum().backward()
    closed = ref.table_gradient([g2, g3], [2, 3], codes.unsqueeze(3), (2, 3, 16, 8))
    torch.testing.assert_close(tables.grad, closed, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(states.grad, g2 + g3)
    for h in range(2):
        rows_codes = codes[:, h].reshape(-1, 3).numpy().astype(np.int32)
        expect = bf.scatter(g2[:, h].reshape(-1, 8).double().numpy(), rows_codes, 3, 16, 2)
        expect += bf.scatter(g3[:, h].reshape(-1, 8).double().numpy(), rows_codes, 3, 16, 3)
        np.testing.assert_allclose(tables.grad[h].double().numpy(), expect, rtol=1e-5, atol=1e-5)
    # invariant: every stage's gradient sums to the summed upstream gradient
    for s in range(3):
        total = sum(g.sum(dim=(0, 2)) for g, e in ((g2, 2), (g3, 3)) if e > s)
        torch.testing.assert_close(tables.grad[:, s].sum(dim=1), total, rtol=1e-4, atol=1e-4)


def test_grouped_cq_matches_bruteforce_and_identity_whitener():
    gen = torch.Generator().manual_seed(5)
    states = ref.synthetic_states(gen, 2, 2, 64, 32, outliers=2)
    books = ref.synthetic_tables(gen, (2, 8, 256, 4), (1.0,), stage_axis=0)
    out, codes, d1, d2 = ref.hard_grouped_cq(states, books, return_margins=True)
    eye = torch.eye(4).repeat(2, 8, 1, 1)
    out_w, codes_w = ref.hard_grouped_cq(states, books, selector_whiteners=eye)
    assert torch.equal(codes, codes_w) and torch.equal(out, out_w)
    x = states.float().reshape(2, 2, 64, 8, 4)
    for h in range(2):
        for g in range(8):
            rows = x[:, h, :, g].reshape(-1, 4).double().numpy()
            bcodes, bd1, bd2 = bf.rvq_encode(rows, books[h, g][None].double().numpy())
            ours = codes[:, h, :, g].reshape(-1).numpy()
            clear = _clear(bd1[:, 0], bd2[:, 0], 1e-5)
            assert np.array_equal(ours[clear], bcodes[clear, 0])
            same = ours == bcodes[:, 0]
            _assert_margins_track(d1[:, h, :, g].reshape(-1).numpy(), d2[:, h, :, g].reshape(-1).numpy(),
                                  bd1[:, 0], bd2[:, 0], same)
    recon = books.half().float()[torch.arange(2)[None, :, None, None], torch.arange(8)[None, None, None, :], codes.long()]
    torch.testing.assert_close(out.float(), recon.reshape(2, 2, 64, 32), rtol=0, atol=0)


def test_whitened_search_matches_bruteforce_in_selector_space():
    gen = torch.Generator().manual_seed(41)
    states = torch.randn(1, 2, 100, 4, generator=gen)
    tables = torch.randn(2, 2, 8, 4, generator=gen)
    w = torch.randn(2, 4, 4, generator=gen)
    _out, codes = ref.hard_residual_vq_exits(states, tables, prefixes=(2,), assignment_whiteners=w)
    for h in range(2):
        xs = (states[0, h].double() @ w[h].double().T).numpy()
        ts = (tables[h].half().double() @ w[h].double().T).numpy()
        bcodes, bd1, bd2 = bf.rvq_encode(xs, ts)
        ours = codes[0, h].numpy()
        clear0 = _clear(bd1[:, 0], bd2[:, 0], 1e-5)
        assert np.array_equal(ours[clear0, 0], bcodes[clear0, 0])


def test_long_whitened_chain_oracle_flips_only_near_ties():
    # 32 whitened full-vector stages (sigma 0.8^s): the fp32 oracle agrees with
    # the float64 search on every code whose float64 margin is clear and flips
    # only near-ties; this floor is what the device kernels are held to there
    stages = 32
    gen = torch.Generator().manual_seed(43 + stages)
    states = ref.synthetic_states(gen, 1, 2, 48, 128)
    tables = ref.synthetic_tables(gen, (2, stages, 256, 128), tuple(0.8 ** s for s in range(stages)), stage_axis=1)
    w = torch.triu(torch.randn(2, 128, 128, generator=gen) * 0.1) + torch.eye(128)
    _out, codes, d1, d2 = ref.hard_residual_vq_exits(states, tables, prefixes=(stages,), assignment_whiteners=w,
                                                     return_margins=True)
    exact, e1, e2 = bruteforce_rvq_codes(states, tables, w)
    res = compare_codes(codes, exact, e1, e2)
    assert res["clear_mismatches"] == 0 and 0.999 < res["agreement"] < 1.0
    # the float64 search itself passes the floor check; a code moved at a
    # clear float64 margin fails it
    assert_codes_with_exact_floor(exact, codes, d1, d2, exact, e1, e2)
    ratio = (e2 - e1) / e1
    n = int(torch.nonzero(ratio[0, 0, :, 0] > 1e-2)[0, 0])
    planted = exact.clone()
    planted[0, 0, n, 0] = (planted[0, 0, n, 0] + 1) % 256
    with pytest.raises(AssertionError):
        assert_codes_with_exact_floor(planted, codes, d1, d2, exact, e1, e2)


def test_grouped_residual_fold_matches_per_group_calls():
    gen = torch.Generator().manual_seed(3)
    states = ref.synthetic_states(gen, 1, 2, 50, 32, outliers=1)
    tables = ref.synthetic_tables(gen, (2, 4, 2, 16, 8), (1.0, 0.5), stage_axis=2)
    out, codes = ref.grouped_residual_vq(states, tables, prefixes=(1, 2))
    for g in range(4):
        sl = slice(8 * g, 8 * g + 8)
        o, c = ref.hard_residual_vq_exits(states[..., sl], tables[:, g], prefixes=(1, 2))
        assert torch.equal(codes[:, :, :, g], c)
        assert torch.equal(out[2][..., sl], o[2])
        assert torch.equal(out[1][..., sl], o[1])


class _Codec:
    def __init__(self, keys, values):
        self.key_tables = [torch.nn.Parameter(k) for k in keys]
        self.value_tables = [torch.nn.Parameter(v) for v in values]


def test_clip_per_layer_kv_reference_expectations():
    # tests/test_pure_uniform16_closed_loop_vq.py:53-77
    codec = _Codec([torch.zeros(1, 16, 2, 2)] * 2, [torch.zeros(1, 16, 2, 2)] * 2)
    codec.key_tables[0].grad = torch.full((1, 16, 2, 2), 2.0)
    codec.value_tables[0].grad = torch.full((1, 16, 2, 2), 0.01)
    codec.key_tables[1].grad = torch.full((1, 16, 2, 2), 0.02)
    codec.value_tables[1].grad = torch.full((1, 16, 2, 2), 0.03)
    audit = ref.clip_codebook_gradients(codec.key_tables, codec.value_tables, maximum_norm=1.0, mode="per_layer_kv")
    rows = {(r["layer"], r["kind"]): r for r in audit["per_group"]}
    assert rows[(0, "key")]["clip_activated"] is True
    assert rows[(0, "key")]["norm_after_clip"] == pytest.approx(1.0)
    assert rows[(0, "value")]["clip_activated"] is False
    assert rows[(0, "value")]["scale"] == pytest.approx(1.0)
    assert rows[(1, "value")]["scale"] == pytest.approx(1.0)


def test_clip_global_and_key_global_reference_expectations():
    # tests/test_pure_uniform16_closed_loop_vq.py:80-123
    codec = _Codec([torch.zeros(1, 16, 2, 2)], [torch.zeros(1, 16, 2, 2)])
    codec.key_tables[0].grad = torch.ones(1, 16, 2, 2)
    codec.value_tables[0].grad = torch.ones(1, 16, 2, 2)
    before = (64 + 64) ** 0.5
    audit = ref.clip_codebook_gradients(codec.key_tables, codec.value_tables, maximum_norm=1.0, mode="global")
    assert audit["total_norm_before_clip"] == pytest.approx(before)
    assert audit["global_scale"] == pytest.approx(1.0 / before)
    both = torch.cat([codec.key_tables[0].grad.flatten(), codec.value_tables[0].grad.flatten()])
    assert torch.linalg.vector_norm(both).item() == pytest.approx(1.0)

    codec = _Codec([torch.zeros(1, 16, 2, 2)] * 2, [torch.zeros(1, 16, 2, 2)] * 2)
    for t, v in zip((*codec.key_tables, *codec.value_tables), (2.0, 3.0, 4.0, 0.01)):
        t.grad = torch.full((1, 16, 2, 2), v)
    audit = ref.clip_codebook_gradients(codec.key_tables, codec.value_tables, maximum_norm=1.0,
                                        mode="key_global_value_per_layer")
    rows = {(r["layer"], r["kind"]): r for r in audit["per_group"]}
    keys = torch.cat([codec.key_tables[0].grad.flatten(), codec.key_tables[1].grad.flatten()])
    assert torch.linalg.vector_norm(keys).item() == pytest.approx(1.0)
    assert rows[(1, "key")]["scale"] == pytest.approx(rows[(0, "key")]["scale"])
    assert rows[(0, "value")]["norm_after_clip"] == pytest.approx(1.0)
    assert rows[(1, "value")]["scale"] == pytest.approx(1.0)


def test_rotary_tables_and_attention_against_fp64():
    pos = torch.arange(0, 5000, 997)
    cos, sin = ref.rotary_cos_sin(pos, 128, 10000.0, dtype=torch.float64)
    i = torch.arange(64, dtype=torch.float64)
    inv = 1.0 / (10000.0 ** (2 * i / 128))
    exact = pos.double()[:, None] * inv[None]
    np.testing.assert_allclose(cos[:, :64].numpy(), np.cos(exact.numpy()), atol=2e-3)
    np.testing.assert_allclose(sin[:, 64:].numpy(), np.sin(exact.numpy()), atol=2e-3)
    # rotation preserves norms per (i, i+64) pair
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(3, 128, generator=gen, dtype=torch.float64)
    c64, s64 = ref.rotary_cos_sin(torch.tensor([5, 77, 4095]), 128, 10000.0, dtype=torch.float64)
    xr = ref.apply_rotary(x, c64, s64)
    pair = x[:, :64] ** 2 + x[:, 64:] ** 2
    pair_r = xr[:, :64] ** 2 + xr[:, 64:] ** 2
    # cos/sin come from fp32 angles and fp32 cos/sin: cos^2+sin^2 = 1 to fp32
    np.testing.assert_allclose(pair.numpy(), pair_r.numpy(), rtol=1e-6)
    # oracle decode step == textbook attention on the rotated fp16 operands
    q = torch.randn(1, 4, 1, 128, generator=gen).half()
    k = torch.randn(1, 1, 50, 128, generator=gen).half()
    v = torch.randn(1, 1, 50, 128, generator=gen).half()
    out = ref.decode_attention(q, k, v, 49, torch.arange(50))
    qc, qs = ref.rotary_cos_sin(torch.tensor([49]), 128, 10000.0)
    kc, ks = ref.rotary_cos_sin(torch.arange(50), 128, 10000.0)
    qr = ref.apply_rotary(q, qc, qs)[0, :, 0]
    kr = ref.apply_rotary(k, kc, ks)[0, 0]
    for hq in range(4):
        row = bf.attention_row(qr[hq].double().numpy(), kr.double().numpy(), v[0, 0].double().numpy())
        np.testing.assert_allclose(out[0, hq, 0].float().numpy(), row, atol=2e-3)


def test_synthetic_generator_is_reproducible():
    a = ref.synthetic_states(torch.Generator().manual_seed(8601), 1, 2, 4, 128)
    b = ref.synthetic_states(torch.Generator().manual_seed(8601), 1, 2, 4, 128)
    assert torch.equal(a, b)
    big = (a.float().abs() > 6).float().mean()
    assert a.dtype == torch.float16 and float(big) < 0.2


def test_prefill_lse_and_value_grad_against_fp64_closed_form():
    # lse: exp(score - lse) over a row's visible keys sums to one and weights
    # the fp64 rows of the attention oracle; dV̂[kvh, s] = sum over the group's
    # heads h and rows t of P[h, t, s] dO[h, t] (the grouping, the mask and the
    # transposition are what a slip here would break)
    gen = torch.Generator().manual_seed(5)
    T, window = 37, 9
    q = torch.randn(2, 4, T, 128, generator=gen).half()
    k = torch.randn(2, 2, T, 128, generator=gen).half()
    v = torch.randn(2, 2, T, 128, generator=gen).half()
    d_out = torch.randn(2, 4, T, 128, generator=gen).half()
    starts = (0, 300)
    lse = ref.prefill_lse(q, k, starts, window=window)
    dv = ref.prefill_value_grad(q, k, v, d_out, starts, window=window)
    mask = ref.sliding_causal_mask(T, window)
    for b in range(2):
        pos = torch.arange(T) + starts[b]
        c, s = ref.rotary_cos_sin(pos, 128, 10000.0)
        qr = ref.apply_rotary(q[b], c[None], s[None]).double()
        kr = ref.apply_rotary(k[b], c[None], s[None]).double()
        expect = torch.zeros(2, T, 128, dtype=torch.float64)
        for hq in range(4):
            scores = qr[hq] @ kr[hq // 2].T / math.sqrt(128)
            p = torch.exp(scores - lse[b, hq].double()[:, None]) * mask
            np.testing.assert_allclose(p.sum(-1).numpy(), 1.0, rtol=1e-5)
            expect[hq // 2] += p.T @ d_out[b, hq].double()
        np.testing.assert_allclose(dv[b].double().numpy(), expect.numpy(), rtol=1e-4, atol=1e-5)


def test_prefill_qk_grad_against_fp64_closed_form():
    # dS = P (dO V^T - rowsum(dO * O)); dq_rot = dS K_rot / sqrt(D) and
    # dk_rot = dS^T Q_rot / sqrt(D) summed over the group; then the rotary's
    # transpose: d_i = r_i cos + r_{i+64} sin, d_{i+64} = r_{i+64} cos - r_i sin
    gen = torch.Generator().manual_seed(6)
    T, window = 29, 11
    q = torch.randn(1, 4, T, 128, generator=gen).half()
    k = torch.randn(1, 2, T, 128, generator=gen).half()
    v = torch.randn(1, 2, T, 128, generator=gen).half()
    d_out = torch.randn(1, 4, T, 128, generator=gen).half()
    dq, dk = ref.prefill_qk_grad(q, k, v, d_out, (70,), window=window)
    pos = torch.arange(T) + 70
    c, s = ref.rotary_cos_sin(pos, 128, 10000.0)
    c, s = c.double(), s.double()
    rot = lambda x: x * c + torch.cat((-x[..., 64:], x[..., :64]), -1) * s
    unrot = lambda r: r * c + torch.cat((r[..., 64:], -r[..., :64]), -1) * s
    mask = ref.sliding_causal_mask(T, window)
    qr, kr = rot(q[0].double()), rot(k[0].double())
    dk_rot = torch.zeros(2, T, 128, dtype=torch.float64)
    for h in range(4):
        scores = (qr[h] @ kr[h // 2].T / math.sqrt(128)).masked_fill(~mask, float("-inf"))
        p = torch.softmax(scores, -1)
        o = p @ v[0, h // 2].double()
        dov = d_out[0, h].double()
        ds = p * (dov @ v[0, h // 2].double().T - (dov * o).sum(-1, keepdim=True))
        np.testing.assert_allclose(dq[0, h].double().numpy(), unrot(ds @ kr[h // 2] / math.sqrt(128)).numpy(),
                                   rtol=1e-4, atol=1e-4)
        dk_rot[h // 2] += ds.T @ qr[h] / math.sqrt(128)
    np.testing.assert_allclose(dk[0].double().numpy(), unrot(dk_rot).numpy(), rtol=1e-4, atol=1e-4)


def test_prefill_oracle_against_fp64_rows_and_masks():
    # the window mask equals torch's is_causal when it does not bind, and each
    # output row equals fp64 textbook attention over its visible keys
    gen = torch.Generator().manual_seed(3)
    mask = ref.sliding_causal_mask(40, 4096)
    assert torch.equal(mask, torch.ones(40, 40, dtype=torch.bool).tril())
    win = ref.sliding_causal_mask(40, 7)
    assert int(win[39].sum()) == 7 and bool(win[39, 33]) and not bool(win[39, 32])
    q = torch.randn(2, 4, 40, 128, generator=gen).half()
    k = torch.randn(2, 2, 40, 128, generator=gen).half()
    v = torch.randn(2, 2, 40, 128, generator=gen).half()
    starts = (0, 1000)
    for window in (4096, 7):
        out = ref.prefill_attention(q, k, v, starts, window=window)
        for b in range(2):
            pos = torch.arange(40) + starts[b]
            c, s = ref.rotary_cos_sin(pos, 128, 10000.0)
            qr = ref.apply_rotary(q[b], c[None], s[None])
            kr = ref.apply_rotary(k[b], c[None], s[None])
            for hq in (0, 3):
                for t in (0, 1, 17, 39):
                    lo = max(0, t - window + 1)
                    row = bf.attention_row(qr[hq, t].double().numpy(), kr[hq // 2, lo : t + 1].double().numpy(),
                                           v[b, hq // 2, lo : t + 1].double().numpy())
                    np.testing.assert_allclose(out[b, hq, t].float().numpy(), row, atol=2e-3)


def test_clear_margin_rule_judges_near_zero_best_distances():
    # a best distance rounded to <= 0 by fp32 cancellation is still a clear
    # winner against a second best far above zero: a different code there fails
    ours = torch.tensor([[1], [2], [3]])
    expect = torch.tensor([[1], [5], [3]])
    d1 = torch.tensor([[1.0], [-1e-6], [2.0]])
    d2 = torch.tensor([[2.0], [0.5], [2.0000001]])
    res = compare_codes(ours, expect, d1, d2)
    assert res["clear_mismatches"] == 1
    # a true near-tie stays exempt
    res = compare_codes(torch.tensor([[4]]), torch.tensor([[3]]), torch.tensor([[2.0]]), torch.tensor([[2.0000001]]))
    assert res["clear_mismatches"] == 0
