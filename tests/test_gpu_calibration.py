"""Codec modules, clip and SGD on the MI355X vs the oracle and the reference's expectations."""

from __future__ import annotations

import pytest
import torch

import jointkv_amd as jkv
from oracle import jointkv_oracle as ref

pytestmark = pytest.mark.gpu


class _Codec:
    def __init__(self, keys, values, device):
        self.key_tables = [torch.nn.Parameter(k.to(device)) for k in keys]
        self.value_tables = [torch.nn.Parameter(v.to(device)) for v in values]


def test_clip_per_layer_kv_expectations(device):
    # tests/test_pure_uniform16_closed_loop_vq.py:53-77
    codec = _Codec([torch.zeros(1, 16, 2, 2)] * 2, [torch.zeros(1, 16, 2, 2)] * 2, device)
    for t, v in zip((codec.key_tables[0], codec.value_tables[0], codec.key_tables[1], codec.value_tables[1]),
                    (2.0, 0.01, 0.02, 0.03)):
        t.grad = torch.full((1, 16, 2, 2), v, device=device)
    audit = jkv.clip_codebook_gradients(codec, maximum_norm=1.0, mode="per_layer_kv")
    assert audit["group_count"] == 4
    rows = {(r["layer"], r["kind"]): r for r in audit["per_group"]}
    assert rows[(0, "key")]["clip_activated"] is True
    assert rows[(0, "key")]["norm_after_clip"] == pytest.approx(1.0)
    assert rows[(0, "value")]["clip_activated"] is False
    assert rows[(0, "value")]["scale"] == pytest.approx(1.0)
    assert rows[(1, "key")]["scale"] == pytest.approx(1.0)
    assert rows[(1, "value")]["scale"] == pytest.approx(1.0)


def test_clip_global_and_key_global(device):
    # tests/test_pure_uniform16_closed_loop_vq.py:80-138
    codec = _Codec([torch.zeros(1, 16, 2, 2)], [torch.zeros(1, 16, 2, 2)], device)
    codec.key_tables[0].grad = torch.ones(1, 16, 2, 2, device=device)
    codec.value_tables[0].grad = torch.ones(1, 16, 2, 2, device=device)
    before = (128) ** 0.5
    audit = jkv.clip_codebook_gradients(codec, maximum_norm=1.0, mode="global")
    assert audit["total_norm_before_clip"] == pytest.approx(before)
    assert audit["global_scale"] == pytest.approx(1.0 / before)
    both = torch.cat([codec.key_tables[0].grad.flatten(), codec.value_tables[0].grad.flatten()])
    assert torch.linalg.vector_norm(both).item() == pytest.approx(1.0)

    codec = _Codec([torch.zeros(1, 16, 2, 2)] * 2, [torch.zeros(1, 16, 2, 2)] * 2, device)
    for t, v in zip((*codec.key_tables, *codec.value_tables), (2.0, 3.0, 4.0, 0.01)):
        t.grad = torch.full((1, 16, 2, 2), v, device=device)
    audit = jkv.clip_codebook_gradients(codec, maximum_norm=1.0, mode="key_global_value_per_layer")
    rows = {(r["layer"], r["kind"]): r for r in audit["per_group"]}
    keys = torch.cat([codec.key_tables[0].grad.flatten(), codec.key_tables[1].grad.flatten()])
    assert audit["group_count"] == 3
    assert torch.linalg.vector_norm(keys).item() == pytest.approx(1.0)
    assert rows[(0, "key")]["shared_group"] == "all_key_tables"
    assert rows[(1, "key")]["scale"] == pytest.approx(rows[(0, "key")]["scale"])
    assert rows[(0, "value")]["norm_after_clip"] == pytest.approx(1.0)
    assert rows[(1, "value")]["scale"] == pytest.approx(1.0)

    codec = _Codec([torch.zeros(1, 16, 2, 2)], [torch.zeros(1, 16, 2, 2)], device)
    codec.key_tables[0].requires_grad_(False)
    codec.value_tables[0].grad = torch.ones(1, 16, 2, 2, device=device)
    audit = jkv.clip_codebook_gradients(codec, maximum_norm=1.0, mode="global")
    assert audit["trainable_group_count"] == 1
    assert codec.key_tables[0].grad is None
    assert torch.linalg.vector_norm(codec.value_tables[0].grad).item() == pytest.approx(1.0)
    with pytest.raises(ValueError, match="unknown gradient clip mode"):
        jkv.clip_codebook_gradients(codec, maximum_norm=1.0, mode="nope")
    with pytest.raises(ValueError, match="finite and positive"):
        jkv.clip_codebook_gradients(codec, maximum_norm=0.0, mode="global")


@pytest.mark.parametrize("mode", ["global", "per_layer_kv", "key_global_value_per_layer"])
def test_clip_matches_oracle_on_random_grads(device, mode):
    gen = torch.Generator().manual_seed(8601)
    keys = [torch.zeros(8, 16, 2, 256, 8) for _ in range(3)]
    values = [torch.zeros(8, 16, 2, 256, 8) for _ in range(3)]
    grads = [torch.randn(8, 16, 2, 256, 8, generator=gen) * s for s in (1e-3, 0.5, 3e-4, 2e-2, 1e-4, 0.7)]
    codec = _Codec(keys, values, device)
    cpu_k = [torch.nn.Parameter(k.clone()) for k in keys]
    cpu_v = [torch.nn.Parameter(v.clone()) for v in values]
    for p, q, g in zip((*codec.key_tables, *codec.value_tables), (*cpu_k, *cpu_v), grads):
        p.grad = g.to(device)
        q.grad = g.clone()
    audit = jkv.clip_codebook_gradients(codec, maximum_norm=1.0, mode=mode)
    expect = ref.clip_codebook_gradients(cpu_k, cpu_v, maximum_norm=1.0, mode=mode)
    for p, q in zip((*codec.key_tables, *codec.value_tables), (*cpu_k, *cpu_v)):
        rel = (p.grad.cpu() - q.grad).norm() / q.grad.norm()
        assert float(rel) <= 1e-5
    assert audit["total_norm_before_clip"] == pytest.approx(expect["total_norm_before_clip"], rel=1e-5)
    assert audit["total_norm_after_clip"] == pytest.approx(expect["total_norm_after_clip"], rel=1e-5)


def test_sgd_step_matches_torch_sgd(device):
    gen = torch.Generator().manual_seed(3)
    params = [torch.nn.Parameter(torch.randn(8, 16, 2, 256, 8, generator=gen).to(device)) for _ in range(2)]
    ref_params = [torch.nn.Parameter(p.detach().clone()) for p in params]
    for p, q in zip(params, ref_params):
        g = torch.randn(p.shape, generator=gen).to(device)
        p.grad = g.clone()
        q.grad = g.clone()
    jkv.sgd_step(params, lr=0.001)
    torch.optim.SGD(ref_params, lr=0.001).step()
    for p, q in zip(params, ref_params):
        torch.testing.assert_close(p.detach(), q.detach(), rtol=1e-6, atol=1e-7)


def test_norms_and_scaled_sgd_on_many_ragged_tensors(device):
    """Over 256 tensors (more than one launch's table), sizes 0 to a few
    thousand that are not multiples of 4, and views 4 bytes off a 16-byte
    boundary: the vector bodies, the scalar tails and the zeroing of every
    output slot."""
    from jointkv_amd import _ops

    gen = torch.Generator().manual_seed(77)
    sizes = [0, 1, 3, 4, 5, 7, 4099, 70001] + [int(torch.randint(0, 3000, (1,), generator=gen)) for _ in range(292)]
    grads, params, cpu_g, cpu_p = [], [], [], []
    for i, n in enumerate(sizes):
        off = i % 2
        g = torch.randn(n + off, generator=gen)
        q = torch.randn(n + off, generator=gen)
        grads.append(g.to(device)[off:])
        params.append(q.to(device)[off:])
        cpu_g.append(g[off:].double())
        cpu_p.append(q[off:])
    norms = _ops.sumsq(grads).cpu()
    expect = torch.stack([(g * g).sum() for g in cpu_g])
    torch.testing.assert_close(norms, expect, rtol=1e-12, atol=1e-12)
    scales = [0.5 + 0.001 * i for i in range(len(sizes))]
    _ops.scale_sgd(grads, scales, params=params, lr=0.01)
    for g, q, g0, q0, sc in zip(grads, params, cpu_g, cpu_p, scales):
        gs = g0.float() * sc
        torch.testing.assert_close(g.cpu(), gs, rtol=0, atol=0)
        torch.testing.assert_close(q.cpu(), q0 - 0.01 * gs, rtol=1e-6, atol=1e-7)


def test_uniform_codec_equals_direct_call_and_v_only_step(device):
    # tests/test_pure_uniform16_closed_loop_vq.py:308-336 relation, on the
    # grouped G2 geometry, then one V-only calibration step (config 5 order:
    # forward -> backward -> finite check -> clip -> SGD).
    gen = torch.Generator().manual_seed(8601)
    k_tab = [ref.synthetic_tables(gen, (8, 16, 2, 256, 8), (1.0, 0.5), stage_axis=2) for _ in range(2)]
    v_tab = [ref.synthetic_tables(gen, (8, 16, 2, 256, 8), (1.0, 0.5), stage_axis=2) for _ in range(2)]
    codec = jkv.ClosedLoopUniformResidualVQ(k_tab, v_tab, [None, None], depth=2, dynamic_bpa=2.0).to(device)
    raw_k = ref.synthetic_states(gen, 1, 8, 128).to(device)
    raw_v = ref.synthetic_states(gen, 1, 8, 128).to(device)
    q = codec(1, raw_k, raw_v)
    ek, ck = jkv.hard_grouped_residual_vq(raw_k, k_tab[1].to(device), prefixes=(2,))
    assert torch.equal(q.key, ek[2]) and torch.equal(q.key_indices, ck)
    assert q.projected_depths is None
    with pytest.raises(ValueError, match="uniform mode"):
        codec(0, raw_k, raw_v, mode="mixed")
    upstream = (torch.randn(q.value.shape, generator=gen) * 1e-3 ** 0.5).half().to(device)
    q.value.backward(upstream)
    assert codec.value_tables[1].grad is not None and codec.key_tables[1].grad is None
    assert bool(torch.isfinite(codec.value_tables[1].grad).all())
    before = codec.value_tables[1].detach().clone()
    grad = codec.value_tables[1].grad.detach().clone()
    audit = jkv.clip_codebook_gradients(codec, maximum_norm=1.0, mode="global")
    jkv.sgd_step(list(codec.value_tables.parameters()), lr=0.001)
    scale = min(1.0, 1.0 / (audit["total_norm_before_clip"] + 1e-6))
    torch.testing.assert_close(codec.value_tables[1].detach(), before - 0.001 * grad * scale, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("grouped,needs", [(True, "tables"), (True, "all"), (False, "all")])
def test_pair_encode_equals_two_encodes(device, grouped, needs):
    # a layer's K and V in one launch (the codec forward's path): the same
    # codes, reconstructions and gradients as two encodes
    print(f"pair encode grouped={grouped} needs={needs}", flush=True)
    gen = torch.Generator().manual_seed(77)
    shape = (8, 16, 2, 256, 8) if grouped else (8, 2, 256, 128)
    stage_axis = 2 if grouped else 1
    tabs = [ref.synthetic_tables(gen, shape, (1.0, 0.5), stage_axis=stage_axis).to(device) for _ in range(2)]
    raw = [ref.synthetic_states(gen, 2, 8, 96).to(device) for _ in range(2)]
    up = [(torch.randn(2, 8, 96, 128, generator=gen) * 1e-2).half().to(device) for _ in range(2)]

    def leaves():
        t = [x.clone().requires_grad_() for x in tabs]
        s = [x.clone().requires_grad_(needs == "all") for x in raw]
        return t, s

    t1, s1 = leaves()
    ek, ck, ev, cv = jkv.closed_loop_vq.hard_residual_vq_pair(s1[0], s1[1], t1[0], t1[1], prefixes=(1, 2))
    (ek[2] * up[0]).float().sum().backward(retain_graph=True)
    ((ev[2] + ev[1]) * up[1]).float().sum().backward()
    t2, s2 = leaves()
    one = jkv.hard_grouped_residual_vq if grouped else jkv.hard_residual_vq_exits
    fk, dk = one(s2[0], t2[0], prefixes=(1, 2))
    fv, dv = one(s2[1], t2[1], prefixes=(1, 2))
    (fk[2] * up[0]).float().sum().backward(retain_graph=True)
    ((fv[2] + fv[1]) * up[1]).float().sum().backward()
    assert torch.equal(ck, dk) and torch.equal(cv, dv)
    assert all(torch.equal(ek[d], fk[d]) and torch.equal(ev[d], fv[d]) for d in (1, 2))
    assert all(torch.equal(a.grad, b.grad) for a, b in zip(t1, t2))
    if needs == "all":
        assert all(torch.equal(a.grad, b.grad) for a, b in zip(s1, s2))
    with pytest.raises(ValueError, match="share their geometry"):
        jkv.closed_loop_vq.hard_residual_vq_pair(raw[0], raw[1][:, :, :5], tabs[0], tabs[1], prefixes=(2,))
    # a frozen K side (the codec's K tables, states without gradient) gives
    # outputs without gradient, as its own encode would: attention above it
    # then forms no key gradient
    vt = tabs[1].clone().requires_grad_()
    ek, _ck, ev, _cv = jkv.closed_loop_vq.hard_residual_vq_pair(raw[0], raw[1], tabs[0], vt, prefixes=(2,))
    assert not ek[2].requires_grad and ev[2].requires_grad


def test_grouped_cq_codec_identity_selector(device):
    gen = torch.Generator().manual_seed(9)
    books_k = [ref.synthetic_tables(gen, (8, 16, 256, 8), (1.0,), stage_axis=0)]
    books_v = [ref.synthetic_tables(gen, (8, 16, 256, 8), (1.0,), stage_axis=0)]
    eye = torch.eye(8).repeat(8, 16, 1, 1)
    codec = jkv.ClosedLoopGroupedCQ(books_k, books_v, [eye], dynamic_bpa=1.0).to(device)
    raw_k = ref.synthetic_states(gen, 1, 8, 64).to(device)
    raw_v = ref.synthetic_states(gen, 1, 8, 64).to(device)
    q = codec(0, raw_k, raw_v)
    # the identity selector is recognised at construction: same kernel and
    # bits as the unwhitened call
    o, c = jkv.hard_grouped_cq(raw_k, books_k[0].to(device))
    assert torch.equal(q.key_indices, c) and torch.equal(q.key, o)
    # the explicitly whitened (generic fp32) path agrees with the oracle to the
    # margin rule; near-ties may resolve differently between the two kernels
    ow, cw = jkv.hard_grouped_cq(raw_k, books_k[0].to(device), selector_whiteners=eye.to(device))
    _r, r_c, d1, d2 = ref.hard_grouped_cq(raw_k.cpu(), books_k[0], selector_whiteners=eye, return_margins=True)
    from parity import assert_codes

    assert_codes(cw[..., None], r_c[..., None], d1[..., None], d2[..., None], agreement=0.999)
    assert_codes(c[..., None], r_c[..., None], d1[..., None], d2[..., None], agreement=0.999)
    with pytest.raises(ValueError, match="one fixed-rate uniform mode"):
        codec(0, raw_k, raw_v, mode="x")


def test_frozen_assignment_reconstruction(device):
    gen = torch.Generator().manual_seed(21)
    tables = torch.randn(2, 16, 5, 3, generator=gen)
    states = torch.randn(1, 2, 7, 3, generator=gen)
    x = states.to(device).requires_grad_()
    t = tables.to(device).requires_grad_()
    exits, codes = jkv.hard_residual_vq_exits(x.detach(), t.detach(), prefixes=(16,))
    out, idx = jkv.frozen_assignment_reconstruction(x, t, codes)
    assert torch.equal(out.detach(), exits[16]) and torch.equal(idx, codes)
    (out.square().mean()).backward()
    assert x.grad is not None and torch.count_nonzero(x.grad) > 0
    assert torch.count_nonzero(t.grad) > 0
    with pytest.raises(ValueError, match="outside codebook"):
        jkv.frozen_assignment_reconstruction(x, t, torch.full((1, 2, 7, 16), 9, device=device))
