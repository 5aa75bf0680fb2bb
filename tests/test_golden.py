"""Golden fixtures (tests/golden/*.npz): the oracle reproduces them, and they
are pinned independently of the oracle by fp64 brute force and closed forms."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bruteforce as bf
from oracle import jointkv_oracle as ref
from tests.parity import assert_codes

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_g2_fixture_oracle_and_bruteforce():
    g = load("g2_encode")
    states = torch.from_numpy(g["states"])
    tables = torch.from_numpy(g["tables_f16"]).float()
    exits, codes, d1, d2 = ref.grouped_residual_vq(states, tables, prefixes=(1, 2), return_margins=True)
    res = assert_codes(codes, torch.from_numpy(g["codes"]), torch.from_numpy(g["d1"]), torch.from_numpy(g["d2"]))
    rows = res["prefix_ok"].all(dim=-1)  # [B,H,T]: every group's codes equal
    assert torch.equal(exits[2][rows], torch.from_numpy(g["exit2"])[rows])
    # independent pin: fp64 exhaustive greedy search per (head, group)
    fx = g["states"].astype(np.float64).reshape(1, 2, 64, 16, 8)
    for h in range(2):
        for grp in (0, 7, 15):
            bcodes, bd1, bd2 = bf.rvq_encode(fx[0, h, :, grp], g["tables_f16"][h, grp].astype(np.float64))
            ours = g["codes"][0, h, :, grp].astype(np.int32)
            clear = (bd2[:, 0] - bd1[:, 0]) > 1e-3 * np.maximum(bd1[:, 0], 1e-30)
            assert np.array_equal(ours[clear, 0], bcodes[clear, 0])
    # exit2 is the fp16 of the fp32 stage sum of the fp16 codewords of the codes
    c = torch.from_numpy(g["codes"]).long()
    t = torch.from_numpy(g["tables_f16"]).float()
    dec = torch.zeros(1, 2, 64, 16, 8)
    for s in range(2):
        for h in range(2):
            dec[0, h] += t[h, torch.arange(16)[None, :], s, c[0, h, :, :, s]]
    assert torch.equal(dec.reshape(1, 2, 64, 128).half(), torch.from_numpy(g["exit2"]))


def test_cq2_fixture_oracle_and_bruteforce():
    g = load("cq2_encode")
    states = torch.from_numpy(g["states"])
    books = torch.from_numpy(g["books_f16"]).float()
    recon, codes, d1, d2 = ref.hard_grouped_cq(states, books, return_margins=True)
    assert_codes(codes[..., None], torch.from_numpy(g["codes"])[..., None], torch.from_numpy(g["d1"])[..., None],
                 torch.from_numpy(g["d2"])[..., None])
    fx = g["states"].astype(np.float64).reshape(1, 2, 64, 32, 4)
    for h in range(2):
        for grp in (0, 31):
            bcodes, bd1, bd2 = bf.rvq_encode(fx[0, h, :, grp], g["books_f16"][h, grp][None].astype(np.float64))
            clear = (bd2[:, 0] - bd1[:, 0]) > 1e-3 * np.maximum(bd1[:, 0], 1e-30)
            assert np.array_equal(g["codes"][0, h, :, grp].astype(np.int32)[clear], bcodes[clear, 0])


def test_scatter_fixture_is_the_exact_bin_sum():
    g = load("scatter")
    codes = torch.from_numpy(g["codes"])
    up = torch.from_numpy(g["upstream"])
    grad = ref.table_gradient([up], [2], codes, (32, 2, 256, 8), accumulate=torch.float64).float().reshape(-1, 8)
    assert torch.equal(grad[torch.from_numpy(g["bin_index"]).long()], torch.from_numpy(g["bin_value"]))
    # every row lands in one bin per stage: the bins sum to the upstream sum
    per = up.double().reshape(2, 16, 16, 8).sum(dim=1)  # [H,G,8]
    bins = torch.zeros(32 * 2 * 256, 8, dtype=torch.float64)
    bins[torch.from_numpy(g["bin_index"]).long()] = torch.from_numpy(g["bin_value"]).double()
    bins = bins.reshape(2, 16, 2, 256, 8).sum(dim=3)
    for s in range(2):
        torch.testing.assert_close(bins[:, :, s], per, rtol=0, atol=1e-6)


def test_attention_fixtures_reproduce():
    g2 = load("g2_encode")
    d = load("decode")
    kt = torch.from_numpy(g2["tables_f16"]).reshape(32, 2, 256, 8).float()
    khat = ref.frozen_decode(torch.from_numpy(d["k_codes"]), kt, 2, torch.float16)
    vhat = ref.frozen_decode(torch.from_numpy(d["v_codes"]), (kt * 0.5).half().float(), 2, torch.float16)
    out = ref.decode_attention(torch.from_numpy(d["q"]), khat, vhat, 79, torch.arange(80))
    assert float((out.float() - torch.from_numpy(d["out"]).float()).abs().max()) <= 1e-3
    p = load("prefill")
    out = ref.prefill_attention(torch.from_numpy(p["q"]), torch.from_numpy(p["k"]), torch.from_numpy(p["v"]),
                                tuple(int(x) for x in p["start"]), window=int(p["window"]))
    assert float((out.float() - torch.from_numpy(p["out"]).float()).abs().max()) <= 1e-3


def test_clip_fixture_closed_form():
    g = load("clip")
    g0, g1 = torch.from_numpy(g["g0"]).double(), torch.from_numpy(g["g1"]).double()
    total = float(torch.sqrt(g0.square().sum() + g1.square().sum()))
    assert float(g["global_norm_before"]) == pytest.approx(total, rel=1e-6)
    coef = min(1.0, 0.5 / (total + 1e-6))
    torch.testing.assert_close(torch.from_numpy(g["global_g0"]).double(), g0 * coef, rtol=1e-6, atol=0)
    for name, gg in (("per_layer_kv_g0", g0), ("per_layer_kv_g1", g1)):
        n = float(torch.linalg.vector_norm(gg))
        torch.testing.assert_close(torch.from_numpy(g[name]).double(), gg * min(1.0, 0.5 / (n + 1e-6)),
                                   rtol=1e-6, atol=0)
