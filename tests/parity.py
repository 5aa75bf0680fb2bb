"""Margin-aware comparison of device results against the oracle."""

from __future__ import annotations

import torch

CODE_MARGIN = 1e-3        # codes bit-exact where (d2-d1)/d1 exceeds this
CODE_AGREEMENT = 0.9999   # overall agreement floor


def compare_codes(ours: torch.Tensor, expect: torch.Tensor, d1: torch.Tensor, d2: torch.Tensor,
                  margin: float = CODE_MARGIN) -> dict:
    """Hierarchical per-vector comparison over the trailing stage axis.

    Stage s of a vector is judged only where stages < s matched (a near-tie
    at an earlier stage legitimately changes every later residual).
    Returns agreement (fraction of judged codes equal) and the number of
    mismatches where the oracle's margin is clear.
    """

    ours = ours.cpu().long()
    expect = expect.cpu().long()
    ratio = (d2.cpu().double() - d1.cpu().double()) / d1.cpu().double().clamp_min(1e-30)
    stages = ours.shape[-1]
    prefix_ok = torch.ones(ours.shape[:-1], dtype=torch.bool)
    judged = equal = clear_bad = 0
    for s in range(stages):
        eq = ours[..., s] == expect[..., s]
        judged += int(prefix_ok.sum())
        equal += int((eq & prefix_ok).sum())
        clear_bad += int((~eq & prefix_ok & (ratio[..., s] > margin)).sum())
        prefix_ok &= eq
    return {
        "agreement": equal / max(judged, 1),
        "clear_mismatches": clear_bad,
        "vectors_fully_equal": float(prefix_ok.float().mean()),
        "prefix_ok": prefix_ok,
    }


def assert_codes(ours, expect, d1, d2, *, agreement=CODE_AGREEMENT):
    res = compare_codes(ours, expect, d1, d2)
    assert res["clear_mismatches"] == 0, f"{res['clear_mismatches']} codes differ at clear margins"
    assert res["agreement"] >= agreement, f"code agreement {res['agreement']:.6f}"
    return res


def assert_recon_rows(ours: torch.Tensor, expect: torch.Tensor, rows_equal: torch.Tensor):
    """Rows whose codes all match must reconstruct within 1e-3 of the row
    norm (the fp16 tolerance); in practice they are bit-identical because
    both sides sum the same fp16 words in fp32 in stage order."""

    ours = ours.detach().cpu().float()
    expect = expect.detach().cpu().float()
    diff = (ours - expect).abs()
    norm = expect.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    rel = diff / norm
    if rows_equal.any():
        assert float(rel[rows_equal].max()) <= 1e-3, "matching codes reconstruct differently"
    return float(diff[rows_equal].max()) if rows_equal.any() else 0.0
