"""Offline gain-shape k-means parent fitting (experiments/
build_frozen_gsrq_multi_exit.py:400-657) on the host: the CPU oracle pinned
by hand-worked sums, exact gain-shape data and the whitened deploy's goal,
and the drop-in's argument checks with the reference's texts."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jointkv_amd import gain_shape
from oracle import gain_shape_oracle as ora
from oracle import jointkv_oracle as ref


def test_codeword_sums_and_update_hand_worked():
    # rows (3,4), (6,8) -> codeword 1 with weights 1 and 0.5; (0,2) -> codeword 0 with weight 2
    rows = np.array([[3.0, 4.0], [6.0, 8.0], [0.0, 2.0]])
    idx = np.array([1, 1, 0])
    w = np.array([1.0, 0.5, 2.0])
    shape_sums, raw_sums, den, _abs = ora.codeword_sums(rows, idx, 3, w)
    np.testing.assert_allclose(shape_sums[1], [0.9, 1.2])      # (0.6, 0.8) * (1 + 0.5)
    np.testing.assert_allclose(raw_sums[1], [6.0, 8.0])        # (3,4) + 0.5 (6,8)
    np.testing.assert_allclose(shape_sums[0], [0.0, 2.0])
    np.testing.assert_allclose(raw_sums[0], [0.0, 4.0])
    np.testing.assert_allclose(den, [2.0, 1.5, 0.0])
    np.testing.assert_allclose(shape_sums[2], [0.0, 0.0])
    shapes0 = np.array([[1.0, 0.0], [1.0, 0.0], [0.0, 1.0]])
    gains0 = np.array([5.0, 5.0, 7.0])
    # without the reserved zero codeword: shape (0.6, 0.8), gain 10 / 1.5;
    # codeword 0: shape (0, 1), gain 4 / 2; the empty codeword 2 keeps its values
    shapes, gains = ora.gskm_update(shapes0, gains0, shape_sums, raw_sums, den, reserve=False)
    np.testing.assert_allclose(shapes, [[0.0, 1.0], [0.6, 0.8], [0.0, 1.0]])
    np.testing.assert_allclose(gains, [2.0, 10.0 / 1.5, 7.0])
    # a cap of 3 binds on codeword 1 and on the untouched codeword 2
    _s, capped = ora.gskm_update(shapes0, gains0, shape_sums, raw_sums, den, cap=3.0, reserve=False)
    np.testing.assert_allclose(capped, [2.0, 3.0, 3.0])
    # the reserved codeword 0 is zero whatever its rows
    shapes_r, gains_r = ora.gskm_update(shapes0, gains0, shape_sums, raw_sums, den, reserve=True)
    assert np.all(shapes_r[0] == 0) and gains_r[0] == 0
    np.testing.assert_allclose(shapes_r[1], [0.6, 0.8])


def test_gain_is_clamped_at_zero():
    # two opposite rows: the summed directions cancel to below 1e-8 -> not
    # updated; one row against the shape: the projection is negative -> gain 0
    rows = np.array([[1.0, 0.0], [-1.0, 0.0], [0.0, 3.0]])
    s_sums, r_sums, den, _abs = ora.codeword_sums(rows, np.array([0, 0, 1]), 2)
    shapes, gains = ora.gskm_update([[0.0, 1.0], [0.0, -1.0]], [4.0, 4.0], s_sums, r_sums, den, reserve=False)
    np.testing.assert_allclose(shapes[0], [0.0, 1.0])
    np.testing.assert_allclose(gains[0], 4.0)
    np.testing.assert_allclose(shapes[1], [0.0, 1.0])
    np.testing.assert_allclose(gains[1], 3.0)
    r_sums[1] = -r_sums[1]
    _s, g = ora.gskm_update([[0.0, 1.0], [0.0, -1.0]], [4.0, 4.0], s_sums, r_sums, den, reserve=False)
    assert g[1] == 0.0


def _exact_clusters(gen, heads, distinct, copies, dim):
    # rows that are exact gain x shape vectors: `distinct` vectors per head,
    # each repeated `copies` times with its own scale
    base = torch.randn(heads, distinct, dim, generator=gen)
    gains = 0.5 + torch.rand(heads, distinct, 1, generator=gen) * 4
    vectors = (base / base.norm(dim=-1, keepdim=True) * gains).float()
    return vectors.repeat_interleave(copies, dim=1).numpy()


def test_fit_of_exact_gain_shape_data():
    # 255 distinct gain-shape vectors, each seeded once: one update leaves
    # every codeword at fp16(gain * shape) of its vector, so the stage's
    # residual is the fp16 rounding error of the data alone
    gen = torch.Generator().manual_seed(5)
    rows = _exact_clusters(gen, 2, 255, 3, 16)
    seeds = [[np.arange(255) * 3 + (h % 3) for h in range(2)]]
    tables, history, _gap = ora.fit_residual_stages(rows, seeds, stages=1, iterations=2)
    want = rows[:, ::3].astype(np.float16)
    np.testing.assert_array_equal(tables[:, 0, 1:], want)
    assert np.all(tables[:, 0, 0] == 0)
    rounding = float(np.square(rows - want.astype(np.float32).repeat(3, axis=1)).mean())
    assert history[0]["residual_element_mse_after"] == pytest.approx(rounding, rel=1e-6)
    assert history[0]["residual_element_mse_after"] < 1e-6 * history[0]["residual_element_mse_before"]
    assert history[0]["occupied_clusters_min"] == 255 and history[0]["zero_assignment_fraction"] == 0.0


def test_whitened_deploy_solves_for_the_selector_goal():
    gen = torch.Generator().manual_seed(6)
    w = (torch.triu(torch.randn(8, 8, generator=gen)) * 0.3 + torch.eye(8) * 2).numpy()
    shapes = torch.nn.functional.normalize(torch.randn(5, 8, generator=gen), dim=-1).numpy()
    gains = np.array([0.0, 1.0, 2.0, 0.5, 3.0])
    raw, sel = ora.deploy(shapes, gains, None, w, "gskm")
    goal = gains[:, None] * shapes
    # the selector image of the fp16-rounded raw word is the goal up to that rounding
    assert np.abs(sel - goal).max() < 4e-3 * np.abs(goal).max()
    np.testing.assert_allclose(sel, raw.astype(np.float64) @ w.T, rtol=1e-6, atol=1e-6)
    # the lower triangle is never read by the solve
    w_low = w + np.tril(np.ones_like(w), -1) * 5
    raw2, _sel2 = ora.deploy(shapes, gains, None, w_low, "gskm")
    np.testing.assert_array_equal(raw2, raw)


def test_fit_invariants_on_clustered_data():
    gen = torch.Generator().manual_seed(7)
    centers = torch.randn(2, 40, 32, generator=gen) * 3
    assign = torch.randint(0, 40, (2, 1200), generator=gen)
    rows = (torch.gather(centers, 1, assign[..., None].expand(-1, -1, 32))
            + 0.3 * torch.randn(2, 1200, 32, generator=gen)).numpy()
    rng = np.random.default_rng(3)
    seeds = [[rng.permutation(1200)[:255] for _ in range(2)] for _ in range(2)]
    caps = np.array([9.0, 12.0])
    tables, history, _gap = ora.fit_residual_stages(rows, seeds, stages=2, iterations=4, caps=caps)
    norms = np.sqrt(np.square(tables.astype(np.float64)).sum(-1))
    assert np.all(tables[:, :, 0] == 0)
    for h in range(2):
        assert norms[h].max() <= caps[h] * (1 + 1e-3)
    for rec in history:
        assert rec["residual_element_mse_after"] < rec["residual_element_mse_before"]
        assert rec["gain_cap_min"] == 9.0 and rec["gain_cap_max"] == 12.0
    # the second stage works on the first stage's residual
    assert history[1]["residual_element_mse_before"] == pytest.approx(history[0]["residual_element_mse_after"])


def test_lloyd_update_is_the_plain_mean_of_each_codewords_rows():
    # build_frozen_gsrq_multi_exit.py:592-603: 255 clusters on a grid 4 apart,
    # each with rows c, c + 2u, c + 4u (u = 0.25 e0) and seeded at c; one
    # update moves every codeword to the rows' mean c + 2u (exact in fp16),
    # which is a fixed point, and codeword 0 stays the reserved zero
    grid = np.stack(np.meshgrid(*[np.arange(1, 5)] * 4, indexing="ij"), -1).reshape(-1, 4)[:255]
    centers = 4.0 * grid.astype(np.float64)
    u = np.array([0.25, 0.0, 0.0, 0.0])
    rows = np.stack([centers, centers + 2 * u, centers + 4 * u], axis=1).reshape(1, 765, 4)
    seeds = [[np.arange(255) * 3]]
    for iterations in (1, 2):
        tables, history, _gap = ora.fit_residual_stages(rows.astype(np.float32), seeds, stages=1,
                                                        iterations=iterations, fit_mode="lloyd")
        assert np.all(tables[0, 0, 0] == 0)
        np.testing.assert_array_equal(tables[0, 0, 1:].astype(np.float64), centers + 2 * u)
        # residuals -2u, 0, +2u along e0: element MSE (0.25 + 0 + 0.25) / 3 / 4
        assert history[0]["residual_element_mse_after"] == pytest.approx(0.5 / 12, rel=1e-12)
        assert history[0]["fit_mode"] == "lloyd" and history[0]["occupied_clusters_min"] == 255


def test_parent_residuals_equal_the_greedy_operator():
    # build_frozen_gsrq_multi_exit.py:661-738 walks the parent's stages with
    # the same greedy search as closed_loop_vq.py:235-410: its reconstruction
    # is the operator's exit (fp16 of the fp32 stage sum) and its residual is
    # what the rows keep after subtracting it, with and without a whitener
    gen = torch.Generator().manual_seed(31)
    states = torch.randn(2, 3, 40, 16, generator=gen).half()
    tables = (torch.randn(3, 3, 256, 16, generator=gen) * torch.tensor([1.0, 0.5, 0.25])[None, :, None, None]).half()
    w = (torch.triu(torch.randn(3, 16, 16, generator=gen)) * 0.2 + torch.eye(16) * 1.5)
    for whitener in (None, w):
        for depth in (1, 3):
            raw, sel, recon, gap = ora.parent_residuals(states.float().numpy(), tables.float().numpy(),
                                                        None if whitener is None else whitener.numpy(), depth)
            exits, codes, d1, d2 = ref.hard_residual_vq_exits(
                states, tables.float(), prefixes=(depth,), assignment_whiteners=whitener, return_margins=True)
            # the inputs keep every search margin clear of fp32 rounding
            assert gap > 1e-5 and float(((d2 - d1) / d1.abs().clamp_min(1e-6)).min()) > 1e-4
            assert torch.equal(torch.from_numpy(recon).half(), exits[depth].detach())
            flat = states.float().permute(1, 0, 2, 3).reshape(3, 80, 16).numpy()
            np.testing.assert_allclose(raw, flat - recon.transpose(1, 0, 2, 3).reshape(3, 80, 16), atol=2e-6)
            if whitener is None:
                assert sel is None
            else:
                want = np.einsum("hde,hne->hnd", whitener.double().numpy(), raw.astype(np.float64))
                np.testing.assert_allclose(sel, want, atol=2e-4)


def test_argument_checks_keep_the_reference_texts():
    residual = torch.zeros(2, 300, 8)
    kw = dict(stages=1, assignment_whiteners=None, initial_selector_residual=None, kmeans_iterations=1,
              token_chunk_size=64, seed=1, fit_mode="gskm", gain_caps=None)
    # no stages: an empty fp16 table before any check
    out, hist = gain_shape.fit_residual_stages(residual, **(kw | {"stages": 0, "fit_mode": "bad"}))
    assert out.shape == (2, 0, 256, 8) and out.dtype == torch.float16 and hist == []
    cases = [
        (dict(sample_weights=-torch.ones(2, 300)), "sample weights must be finite non-negative"),
        (dict(sample_weights=torch.ones(2, 299)), "sample weights must be finite non-negative"),
        (dict(sample_weights=torch.cat([torch.ones(1, 300), torch.zeros(1, 300)])), "positive mass"),
        (dict(fit_mode="kmeans"), "extension fit mode must be gskm or lloyd"),
        (dict(initial_selector_residual=residual), "selector residual requires assignment whiteners"),
        (dict(assignment_whiteners=torch.eye(8).expand(2, 8, 8)),
         "whitened extension requires the exact parent selector residual"),
        (dict(assignment_whiteners=torch.eye(8).expand(2, 8, 8), initial_selector_residual=residual[:, :10]),
         "raw/selector parent residual geometry differs"),
        (dict(gain_caps=torch.tensor([1.0, 0.0])), "extension gain caps must be finite positive"),
        (dict(gain_caps=torch.tensor([1.0])), "extension gain caps must be finite positive"),
        (dict(token_chunk_size=0), "token chunk size must be positive"),
    ]
    for extra, text in cases:
        with pytest.raises(ValueError, match=text):
            gain_shape.fit_residual_stages(residual, **(kw | extra))
    with pytest.raises(ValueError, match="at least 255 rows"):
        gain_shape.fit_residual_stages(residual[:, :200], **kw)
    with pytest.raises(ValueError, match="state/centroid geometry differs"):
        gain_shape.nearest_indices(residual, torch.zeros(2, 4, 7), assignment_whiteners=None, token_chunk_size=8)
