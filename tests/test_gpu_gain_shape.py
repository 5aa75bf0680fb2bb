"""Gain-shape k-means parent fitting on the MI355X (experiments/
build_frozen_gsrq_multi_exit.py:400-657): the per-codeword sums and the
residual update against the CPU oracle, and whole fits against the oracle
run on the same seed rows."""

from __future__ import annotations

import time

import numpy as np
import pytest
import torch

from jointkv_amd import _ops, gain_shape
from oracle import gain_shape_oracle as ora

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("heads,rows,dim,weighted", [
    (3, 400, 128, False),   # one slice: each codeword's sum runs in row order
    (3, 400, 37, True),     # odd width, weighted
    (4, 5000, 64, False),   # several slices
    (2, 70000, 128, True),  # many slices, weighted
])
def test_gain_shape_sums_match_oracle(device, heads, rows, dim, weighted):
    print(f"gain-shape sums H={heads} N={rows} D={dim} weighted={weighted}", flush=True)
    gen = torch.Generator().manual_seed(rows + dim)
    x = torch.randn(heads, rows, dim, generator=gen) * 2
    idx = torch.randint(0, 250, (heads, rows), generator=gen)  # codewords 250..255 stay empty
    idx[:, ::7] = 5                                            # one crowded codeword
    w = torch.rand(heads, rows, generator=gen) if weighted else None
    args = (x.to(device), idx.to(device), 256)
    kw = dict(weights=None if w is None else w.to(device))
    shape, raw, den = _ops.gain_shape_sums(*args, **kw)
    again = _ops.gain_shape_sums(*args, **kw)
    assert all(torch.equal(a, b) for a, b in zip((shape, raw, den), again)), "sums differ between runs"
    for h in range(heads):
        s, r, d, a = ora.codeword_sums(x[h].numpy(), idx[h].numpy(), 256, None if w is None else w[h].numpy())
        # fp32 sums of up to a few thousand terms against float64
        assert np.all(np.abs(raw[h].cpu().double().numpy() - r) <= 2e-5 * a + 1e-6)
        assert np.all(np.abs(shape[h].cpu().double().numpy() - s) <= 2e-5 * d[:, None] + 1e-6)
        np.testing.assert_allclose(den[h].cpu().double().numpy(), d, rtol=1e-5, atol=0)
        assert not raw[h, 250:].any() and not den[h, 250:].any()
    if w is None:
        # integer counts are exact
        assert torch.equal(den.cpu(), torch.stack([torch.bincount(i, minlength=256) for i in idx]).float())
    if rows == 400 and w is None:
        # a single slice sums each codeword in row order: torch's CPU index_add_, bit for bit
        want = torch.stack([torch.zeros(256, dim).index_add_(0, idx[h], x[h]) for h in range(heads)])
        assert torch.equal(raw.cpu(), want)
    # without shapes only the plain sums and the weights
    none, raw2, den2 = _ops.gain_shape_sums(*args, weights=kw["weights"], with_shapes=False)
    assert none is None and torch.equal(raw2, raw) and torch.equal(den2, den)


def test_subtract_codewords(device):
    gen = torch.Generator().manual_seed(31)
    res = torch.randn(2, 1000, 128, generator=gen)
    tab = torch.randn(2, 256, 128, generator=gen)
    idx = torch.randint(0, 256, (2, 1000), generator=gen)
    idx[0, 3], idx[1, 7] = -1, 256  # no codeword: rows left as they are
    want = res.clone()
    ok = (idx >= 0) & (idx < 256)
    want[ok] -= torch.gather(tab, 1, idx.clamp(0, 255)[..., None].expand(-1, -1, 128))[ok]
    got = res.to(device)
    _ops.subtract_codewords(got, tab.to(device), idx.to(device))
    assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("mode,weighted,capped,reserve", [
    ("gskm", False, False, True), ("gskm", True, True, True), ("gskm", True, False, False),
    ("lloyd", False, False, True), ("lloyd", False, False, False),
])
def test_lloyd_update_matches_oracle(device, mode, weighted, capped, reserve):
    # one update from a given assignment with crowded, single-row and empty
    # codewords (the whole-fit tests below have one row per codeword)
    print(f"update mode={mode} weighted={weighted} capped={capped} reserve={reserve}", flush=True)
    gen = torch.Generator().manual_seed(123)
    heads, rows, dim, k = 2, 3000, 128, 256
    work = torch.randn(heads, rows, dim, generator=gen) * 3
    raw_rows = torch.randn(heads, rows, dim, generator=gen) * 2
    idx = torch.randint(0, 200, (heads, rows), generator=gen)   # 200..255 empty
    idx[:, :50] = 7                                             # a crowded codeword
    idx[0, 60], idx[1, 61] = 201, 202                           # single rows
    shapes = torch.nn.functional.normalize(torch.randn(heads, k, dim, generator=gen), dim=-1)
    gains = torch.rand(heads, k, generator=gen) * 5
    means = torch.randn(heads, k, dim, generator=gen)
    weights = torch.rand(heads, rows, generator=gen) + 0.1 if weighted else None
    caps = torch.tensor([4.0, 2.5]) if capped else None
    stage = gain_shape._Stage(mode, None, gains.to(device).clone(), shapes.to(device).clone(),
                              means.to(device).clone(), None if caps is None else caps.to(device), reserve)
    stage.update(work.to(device), raw_rows.to(device), idx.to(device), None if weights is None else weights.to(device))
    for h in range(heads):
        w_h = None if weights is None else weights[h].numpy()
        if mode == "gskm":
            ss, rs, den, _a = ora.codeword_sums(work[h].numpy(), idx[h].numpy(), k, w_h)
            want_s, want_g = ora.gskm_update(shapes[h].numpy(), gains[h].numpy(), ss, rs, den,
                                             None if caps is None else float(caps[h]), reserve)
            np.testing.assert_allclose(stage.shapes[h].cpu().double().numpy(), want_s, rtol=0, atol=2e-6)
            np.testing.assert_allclose(stage.gains[h].cpu().double().numpy(), want_g, rtol=1e-5, atol=1e-6)
        else:
            _ss, rs, den, _a = ora.codeword_sums(raw_rows[h].numpy(), idx[h].numpy(), k)
            ok = den > 0
            if reserve:
                ok[0] = False
            want = means[h].double().numpy().copy()
            want[ok] = rs[ok] / den[ok, None]
            if reserve:
                want[0] = 0.0
            np.testing.assert_allclose(stage.means[h].cpu().double().numpy(), want, rtol=0, atol=2e-6)


def _seed_rows_only(gen, heads, rows, dim):
    # as many distinct rows as seeds, each with its own scale: every row is a
    # codeword's seed, so every search of every stage has a wide margin (a
    # row's own codeword against the others) and the device's and the
    # oracle's runs make the same choices throughout
    x = torch.randn(heads, rows, dim, generator=gen)
    return (x * (0.5 + 2 * torch.rand(heads, rows, 1, generator=gen))).float()


def _device_seeds(device, seed, stages, heads, rows, picks):
    """The seed rows the drop-in draws: one permutation per head per stage
    from a generator on the device."""

    g = torch.Generator(device=device).manual_seed(seed)
    return [[torch.randperm(rows, generator=g, device=device)[:picks].cpu().numpy() for _ in range(heads)]
            for _ in range(stages)]


@pytest.mark.parametrize("mode,whitened,weighted,capped,reserve", [
    ("gskm", False, False, False, True),
    ("gskm", True, True, True, True),
    ("gskm", False, True, False, False),
    ("lloyd", True, False, False, True),
    ("lloyd", False, False, False, False),
])
def test_fit_matches_oracle(device, mode, whitened, weighted, capped, reserve):
    print(f"fit mode={mode} whitened={whitened} weighted={weighted} capped={capped} reserve={reserve}",
          flush=True)
    heads, dim, stages, iterations, seed = 2, 128, 2, 3, 9301
    rows = 255 if reserve else 256
    gen = torch.Generator().manual_seed(77)
    residual = _seed_rows_only(gen, heads, rows, dim)
    w = (torch.triu(torch.randn(heads, dim, dim, generator=gen)) * 0.05
         + torch.eye(dim) * 1.5) if whitened else None
    selector = torch.matmul(residual, w.transpose(-1, -2)) if whitened else None
    weights = 0.2 + torch.rand(heads, rows, generator=gen) if weighted else None
    caps = torch.tensor([10.0, 14.0]) if capped else None
    picks = 255 if reserve else 256
    seeds = _device_seeds(device, seed, stages, heads, rows, picks)
    dev_res = residual.to(device)
    got, hist = gain_shape.fit_residual_stages(
        dev_res, stages=stages, assignment_whiteners=None if w is None else w.to(device),
        initial_selector_residual=None if selector is None else selector.to(device),
        sample_weights=None if weights is None else weights.to(device), kmeans_iterations=iterations,
        token_chunk_size=4096, seed=seed, fit_mode=mode, gain_caps=None if caps is None else caps.to(device),
        reserve_zero_codeword=reserve)
    assert got.dtype == torch.float16 and got.device.type == "cpu" and got.shape == (heads, stages, 256, dim)
    # the oracle on the same seed rows; each of its stages ends with the
    # device's table, so the next stage starts from the same residual
    want, want_hist, margin = ora.fit_residual_stages(
        residual.numpy(), seeds, stages=stages, whitener=None if w is None else w.numpy(),
        selector_residual=None if selector is None else selector.numpy(),
        weights=None if weights is None else weights.numpy(), iterations=iterations, fit_mode=mode,
        caps=None if caps is None else caps.numpy(), reserve=reserve, forced_tables=got.numpy())
    # the premise: no search of the oracle's run lies within rounding of a tie
    assert margin > 1e-4, margin
    g = got.float().numpy()
    t = want.astype(np.float32)
    # fp32 device sums against float64: at most one fp16 step apart, and
    # rarely even that in the first stage (the second stage's residuals
    # x - fp16(x) often sit exactly on an fp16 midpoint, where the last fp32
    # bit of gain x shape decides the rounding)
    step = np.maximum(np.spacing(np.abs(want)), np.spacing(np.abs(got.numpy()))).astype(np.float32)
    if whitened:
        # plus the fp32 triangular solve's error, which scales with the row;
        # later stages fit the selector residual left by an fp32 product
        # (x W^T less fp16(raw) W^T), whose rounding is about 1e-3 of that
        # residual's own size here
        rowmax = np.abs(t).max(axis=-1, keepdims=True)
        step = step + rowmax * np.array([1e-4] + [1e-2] * (stages - 1), dtype=np.float32)[None, :, None, None]
    assert np.all(np.abs(g - t) <= step), float((np.abs(g - t) / step).max())
    assert float((g[:, 0] != t[:, 0]).mean()) < 0.01
    assert len(hist) == stages
    for ours, ref in zip(hist, want_hist):
        assert set(ours) == set(ref)
        for key, value in ref.items():
            if isinstance(value, float):
                assert ours[key] == pytest.approx(value, rel=1e-5, abs=1e-9), key
            else:
                assert ours[key] == value, key
    # the residual was updated in place
    assert hist[-1]["residual_element_mse_after"] == pytest.approx(float(dev_res.square().mean()), rel=1e-6)


@pytest.mark.parametrize("whitened", [False, True])
def test_parent_residuals_match_oracle(device, whitened):
    # the frozen parent's exit residuals: greedy nearest (selector) words,
    # subtracted from the raw residual and summed into the reconstruction
    print(f"parent residuals whitened={whitened}", flush=True)
    gen = torch.Generator().manual_seed(408)
    states = torch.randn(2, 2, 150, 128, generator=gen).half()
    tables = torch.stack([torch.randn(2, 256, 128, generator=gen) * s for s in (1.0, 0.5, 0.25)], dim=1).half()
    w = (torch.triu(torch.randn(2, 128, 128, generator=gen)) * 0.05 + torch.eye(128) * 1.5) if whitened else None
    raw, sel, recon = gain_shape.parent_residuals_and_reconstruction(
        states.to(device), tables.to(device), None if w is None else w.to(device), depth=2, token_chunk_size=4096)
    want_raw, want_sel, want_recon, margin = ora.parent_residuals(
        states.float().numpy(), tables.float().numpy(), None if w is None else w.numpy(), 2)
    # an fp32 distance over 128 dims errs by at most 128 eps |x||c|, under
    # 4e-6 of |x|^2 + |c|^2 for either side: a wider gap cannot flip
    assert margin > 1e-5, margin
    # same choices: the same fp32 subtractions and sums, bit for bit
    assert np.array_equal(raw.cpu().numpy(), want_raw)
    assert recon.dtype == torch.float16 and torch.equal(recon.cpu(), torch.from_numpy(want_recon).half())
    if whitened:
        np.testing.assert_allclose(sel.cpu().numpy(), want_sel, rtol=0, atol=2e-4 * np.abs(want_sel).max())
    else:
        assert sel is None


def test_fit_config_size_properties(device):
    # a calibration-sized fit: 8 heads, 32768 rows, head dim 128, ten Lloyd
    # iterations per stage, two stages, gradient weights and gain caps
    gen = torch.Generator(device=device).manual_seed(5)
    heads, rows, dim = 8, 32768, 128
    centers = torch.randn(heads, 512, dim, generator=gen, device=device)
    pick = torch.randint(0, 512, (heads, rows), generator=gen, device=device)
    residual = torch.gather(centers, 1, pick[..., None].expand(-1, -1, dim)) + 0.3 * torch.randn(
        heads, rows, dim, generator=gen, device=device)
    weights = 0.5 + torch.rand(heads, rows, generator=gen, device=device)
    caps = torch.full((heads,), 20.0, device=device)
    kw = dict(stages=2, assignment_whiteners=None, initial_selector_residual=None, sample_weights=weights,
              kmeans_iterations=10, token_chunk_size=4096, seed=11, fit_mode="gskm", gain_caps=caps)
    first = residual.clone()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tables, hist = gain_shape.fit_residual_stages(first, **kw)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    print(f"  fit H={heads} N={rows} D={dim}, 2 stages x 10 iterations: {elapsed * 1e3:.0f} ms", flush=True)
    for rec in hist:
        print(f"  stage {rec['stage']}: mse {rec['residual_element_mse_before']:.4f} -> "
              f"{rec['residual_element_mse_after']:.4f}, occupied >= {rec['occupied_clusters_min']}", flush=True)
        assert rec["residual_element_mse_after"] < rec["residual_element_mse_before"]
        assert rec["occupied_clusters_min"] >= 200 and rec["gradient_weighted"] == 1
        assert rec["maximum_codeword_norm"] <= 20.0 * (1 + 2 ** -10)
    assert torch.isfinite(tables.float()).all() and not tables[:, :, 0].float().any()
    # the same seed gives the same tables, bit for bit
    second = residual.clone()
    tables2, _hist2 = gain_shape.fit_residual_stages(second, **kw)
    assert torch.equal(tables, tables2) and torch.equal(first, second)
