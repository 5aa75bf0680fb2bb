"""The HIP path on the golden fixtures' inputs against their expected outputs."""

from __future__ import annotations

import pytest
import torch

import jointkv_amd as jkv
from jointkv_amd import _ops
from tests.parity import assert_codes, assert_recon_rows
from tests.test_golden import load

pytestmark = pytest.mark.gpu


def test_golden_g2_encode(device):
    g = load("g2_encode")
    states = torch.from_numpy(g["states"]).to(device)
    tables = torch.from_numpy(g["tables_f16"]).float().to(device)
    exits, codes = jkv.hard_grouped_residual_vq(states, tables, prefixes=(1, 2))
    res = assert_codes(codes.cpu(), torch.from_numpy(g["codes"]), torch.from_numpy(g["d1"]),
                       torch.from_numpy(g["d2"]))
    rows = res["prefix_ok"].all(dim=-1)
    assert_recon_rows(exits[2], torch.from_numpy(g["exit2"]), rows)
    assert torch.equal(exits[2].cpu()[rows], torch.from_numpy(g["exit2"])[rows])


def test_golden_cq2_encode(device):
    g = load("cq2_encode")
    recon, codes = jkv.hard_grouped_cq(torch.from_numpy(g["states"]).to(device),
                                       torch.from_numpy(g["books_f16"]).float().to(device))
    res = assert_codes(codes.cpu()[..., None], torch.from_numpy(g["codes"])[..., None],
                       torch.from_numpy(g["d1"])[..., None], torch.from_numpy(g["d2"])[..., None])
    rows = res["prefix_ok"].all(dim=-1)
    assert torch.equal(recon.cpu()[rows], torch.from_numpy(g["recon"])[rows])


def test_golden_scatter(device):
    g = load("scatter")
    grad = torch.zeros(32, 2, 256, 8, device=device)
    _ops.rvq_scatter_grad([torch.from_numpy(g["upstream"]).to(device)], [2],
                          torch.from_numpy(g["codes"]).to(device), grad, group_dim=8)
    flat = grad.cpu().reshape(-1, 8)
    idx = torch.from_numpy(g["bin_index"]).long()
    assert torch.equal(flat[idx], torch.from_numpy(g["bin_value"]))
    mask = torch.ones(flat.shape[0], dtype=torch.bool)
    mask[idx] = False
    assert int(flat[mask].count_nonzero()) == 0


def test_golden_decode_and_prefill(device):
    g2 = load("g2_encode")
    d = load("decode")
    kt = torch.from_numpy(g2["tables_f16"]).reshape(32, 2, 256, 8)
    vt = (kt.float() * 0.5).half()
    out = jkv.decode_attention(torch.from_numpy(d["q"]).to(device), torch.from_numpy(d["k_codes"]).to(device),
                               torch.from_numpy(d["v_codes"]).to(device), kt.to(device), vt.to(device),
                               torch.tensor([80], dtype=torch.int32, device=device))
    assert float((out.cpu().float() - torch.from_numpy(d["out"]).float()).abs().max()) <= 2e-3
    p = load("prefill")
    out = jkv.prefill_attention(torch.from_numpy(p["q"]).to(device), torch.from_numpy(p["k"]).to(device),
                                torch.from_numpy(p["v"]).to(device), [int(x) for x in p["start"]],
                                window=int(p["window"]))
    assert float((out.cpu().float() - torch.from_numpy(p["out"]).float()).abs().max()) <= 2e-3


def test_golden_clip(device):
    g = load("clip")

    class Codec:
        key_tables = []
        value_tables = []

    for mode in ("global", "per_layer_kv"):
        Codec.value_tables = [torch.nn.Parameter(torch.zeros(2, 2, 64, 8, device=device)) for _ in range(2)]
        for p, name in zip(Codec.value_tables, ("g0", "g1")):
            p.grad = torch.from_numpy(g[name]).to(device)
        audit = jkv.clip_codebook_gradients(Codec, maximum_norm=0.5, mode=mode)
        assert audit["total_norm_before_clip"] == pytest.approx(float(g[f"{mode}_norm_before"]), rel=1e-6)
        for p, name in zip(Codec.value_tables, ("g0", "g1")):
            torch.testing.assert_close(p.grad.cpu(), torch.from_numpy(g[f"{mode}_{name}"]), rtol=1e-6, atol=0)
