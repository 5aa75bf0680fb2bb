"""Offline gain-shape k-means parent fitting on gfx950 kernels.

Drop-in for ``nearest_indices``, ``fit_residual_stages`` and
``parent_residuals_and_reconstruction`` of
``experiments/build_frozen_gsrq_multi_exit.py`` (:364-397, :400-657,
:661-738): the residual stages that extend a frozen parent codec, fitted in
the parent's deployed metric, and the parent's residuals they start from.

Each stage keeps, per head, K codewords as a non-negative gain times a unit
shape (``fit_mode="gskm"``) or as plain Lloyd means (``"lloyd"``).  A Lloyd
iteration is

  deploy (fp16 round trip of gain x shape, through the whitener's triangular
  solve when there is one) -> nearest codeword of every working row
  (``jkv_nearest_f32``) -> per-codeword sums of the rows, their unit
  directions and the weights in one pass (``jkv_gain_shape_sums``) ->
  shape = direction of the summed unit rows, gain = mean projection of the
  rows on it, clamped to [0, cap].

After the iterations the stage's codewords are subtracted from the raw (and
selector) residual of every row (``jkv_subtract_codewords``).  The per-head
work is batched over all heads; only the [H,K,D] codeword updates, the
seeding and the whitener's small triangular solves are PyTorch ops.

Seeding draws the same ``torch.randperm`` sequence from a generator on the
residual's device as the reference does (per stage, head by head), so a run
on the same device type starts from the same rows.
"""

from __future__ import annotations

from typing import Any

import torch
import torch.nn.functional as F

from . import _ops

CLUSTERS = 256  # codewords per stage (8-bit stages)


def _check_chunk(token_chunk_size: int) -> None:
    if int(token_chunk_size) <= 0:
        raise ValueError("token chunk size must be positive")


@torch.no_grad()
def nearest_indices(
    states: torch.Tensor,
    centroids: torch.Tensor,
    *,
    assignment_whiteners: torch.Tensor | None,
    token_chunk_size: int,
) -> torch.Tensor:
    """Nearest centroid of every row (build_frozen_gsrq_multi_exit.py:364-397).

    ``states[H,N,D]``, ``centroids[H,K,D]``; with ``assignment_whiteners``
    ``[H,D,D]`` both are mapped to ``W x`` first.  Distances are
    ``(|x|^2 + |c|^2) - 2 x.c`` in fp32, the lowest index on ties; returns
    int64 ``[H,N]``.  One HIP launch covers every row: ``token_chunk_size``
    is validated and otherwise unused.
    """

    heads, _tokens, dimension = states.shape
    if centroids.shape[0] != heads or centroids.shape[2] != dimension:
        raise ValueError("state/centroid geometry differs")
    _check_chunk(token_chunk_size)
    states = states.float()
    centroids = centroids.float()
    if assignment_whiteners is not None:
        wt = assignment_whiteners.float().transpose(-1, -2).contiguous()
        states = torch.matmul(states, wt)
        centroids = torch.matmul(centroids, wt)
    return _ops.nearest_f32(states, centroids)


@torch.no_grad()
def parent_residuals_and_reconstruction(
    states: torch.Tensor,
    tables: torch.Tensor,
    whitener: torch.Tensor | None,
    *,
    depth: int,
    token_chunk_size: int,
) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor]:
    """The frozen parent's exact residuals at exit ``depth``
    (build_frozen_gsrq_multi_exit.py:661-738).

    ``states[B,H,T,D]``, parent ``tables[H,S,K,D]`` (deployed values),
    ``whitener[H,D,D]`` or None.  Greedy stage by stage: nearest (selector)
    codeword of the residual, whose raw word is subtracted from the raw
    residual and added to the reconstruction (and whose selector word is
    subtracted from the selector residual).  Returns the raw residual
    ``[H,B*T,D]`` fp32, the selector residual (or None) and the
    reconstruction ``[B,H,T,D]`` in the states' dtype.
    """

    batch, heads, tokens, dimension = states.shape
    _check_chunk(token_chunk_size)
    flat = states.permute(1, 0, 2, 3).reshape(heads, batch * tokens, dimension).float()
    raw_residual = flat.clone()
    negated = torch.zeros_like(raw_residual)  # minus the reconstruction: exact negation of the running sum
    selector_residual = None
    raw_tables = tables[:, :depth].to(device=states.device, dtype=torch.float32)
    selector_tables = raw_tables
    if whitener is not None:
        w = whitener.to(device=states.device, dtype=torch.float32)
        wt = w.transpose(-1, -2).contiguous()
        selector_residual = torch.matmul(flat, wt).contiguous()
        selector_tables = torch.matmul(raw_tables, wt.unsqueeze(1))
    for stage in range(depth):
        raw_table = raw_tables[:, stage].contiguous()
        selector_table = selector_tables[:, stage].contiguous()
        indices = _ops.nearest_f32(raw_residual if selector_residual is None else selector_residual,
                                   selector_table)
        _ops.subtract_codewords(negated, raw_table, indices)
        _ops.subtract_codewords(raw_residual, raw_table, indices)
        if selector_residual is not None:
            _ops.subtract_codewords(selector_residual, selector_table, indices)
    reconstruction = (-negated).reshape(heads, batch, tokens, dimension).permute(1, 0, 2, 3).to(
        states.dtype).contiguous()
    return raw_residual, selector_residual, reconstruction


def _validate(residual, sample_weights, fit_mode, assignment_whiteners, initial_selector_residual, gain_caps):
    """The reference's checks, in its order and with its texts (:434-470)."""

    heads, tokens, _dimension = residual.shape
    if sample_weights is not None:
        sample_weights = sample_weights.to(device=residual.device, dtype=torch.float32)
        if (tuple(sample_weights.shape) != (heads, tokens) or not bool(torch.isfinite(sample_weights).all())
                or bool((sample_weights < 0).any()) or bool((sample_weights.sum(dim=1) <= 0).any())):
            raise ValueError("sample weights must be finite non-negative [H,N] with "
                             "positive mass for every head")
    if fit_mode not in {"gskm", "lloyd"}:
        raise ValueError("extension fit mode must be gskm or lloyd")
    if assignment_whiteners is None:
        if initial_selector_residual is not None:
            raise ValueError("selector residual requires assignment whiteners")
    else:
        if initial_selector_residual is None:
            raise ValueError("whitened extension requires the exact parent selector residual")
        if initial_selector_residual.shape != residual.shape:
            raise ValueError("raw/selector parent residual geometry differs")
    if gain_caps is not None:
        gain_caps = gain_caps.to(device=residual.device, dtype=torch.float32)
        if (tuple(gain_caps.shape) != (heads,) or not bool(torch.isfinite(gain_caps).all())
                or bool((gain_caps <= 0).any())):
            raise ValueError("extension gain caps must be finite positive [H]")
    return sample_weights, gain_caps


class _Stage:
    """One stage's codewords: gain x unit shape (gskm) or free means (lloyd)."""

    def __init__(self, fit_mode, whitener, gains, shapes, means, caps, reserve):
        self.fit_mode = fit_mode
        self.whitener = whitener
        self.gains, self.shapes, self.means = gains, shapes, means
        self.caps = caps
        self.reserve = reserve

    def deployed(self) -> tuple[torch.Tensor, torch.Tensor]:
        """fp16-rounded raw codewords and their selector images, fp32 [H,K,D]."""

        if self.fit_mode == "gskm":
            selector_goal = self.shapes * self.gains.unsqueeze(-1)
            if self.whitener is None:
                raw = selector_goal
            else:
                # raw = goal W^-T: W (upper triangular) times raw^T = goal^T
                raw = torch.linalg.solve_triangular(self.whitener, selector_goal.transpose(-1, -2),
                                                    upper=True).transpose(-1, -2)
        else:
            raw = self.means
        raw = raw.half().float()
        selector = raw if self.whitener is None else torch.matmul(raw, self.whitener.transpose(-1, -2))
        return raw.contiguous(), selector.contiguous()

    def update(self, working, raw_rows, indices, weights) -> None:
        """One Lloyd update from the current assignment."""

        clusters = int(self.means.shape[1] if self.fit_mode == "lloyd" else self.shapes.shape[1])
        if self.fit_mode == "lloyd":
            # plain means of the raw rows; the weights do not enter
            _none, sums, counts = _ops.gain_shape_sums(raw_rows, indices, clusters, with_shapes=False)
            keep = counts > 0
            if self.reserve:
                keep[:, 0] = False
            self.means = torch.where(keep.unsqueeze(-1), sums / counts.clamp_min(1.0).unsqueeze(-1), self.means)
            if self.reserve:
                self.means[:, 0] = 0.0
            return
        directions, sums, mass = _ops.gain_shape_sums(working, indices, clusters, weights=weights)
        length = torch.linalg.vector_norm(directions, dim=-1)
        keep = (mass > 0) & (length > 1e-8)
        if self.reserve:
            keep[:, 0] = False
        unit = directions / torch.where(keep, length, torch.ones_like(length)).unsqueeze(-1)
        self.shapes = torch.where(keep.unsqueeze(-1), unit, self.shapes)
        # the mean projection of the rows on the new shape
        projection = (sums * self.shapes).sum(dim=-1)
        gain = (projection / torch.where(keep, mass, torch.ones_like(mass))).clamp_min(0.0)
        self.gains = torch.where(keep, gain, self.gains)
        if self.caps is not None:
            self.gains = torch.minimum(self.gains, self.caps.unsqueeze(-1))
        if self.reserve:
            self.shapes[:, 0] = 0.0
            self.gains[:, 0] = 0.0


def _seed_stage(generator, working, raw_rows, fit_mode, reserve, caps, whitener) -> _Stage:
    """K seeds per head from distinct random rows (:478-510): the first
    255 (or 256) rows of a fresh permutation, head by head, plus the zero
    codeword in slot 0 when it is reserved."""

    heads, tokens, dimension = working.shape
    picks = 255 if reserve else 256
    chosen = torch.stack([torch.randperm(tokens, generator=generator, device=working.device)[:picks]
                          for _ in range(heads)])
    gather = chosen.unsqueeze(-1).expand(-1, -1, dimension)
    sampled = torch.gather(working, 1, gather)
    gains = torch.linalg.vector_norm(sampled, dim=-1)
    if fit_mode == "gskm":
        seeds = F.normalize(sampled, dim=-1, eps=1e-8)
    else:
        seeds = torch.gather(raw_rows, 1, gather)
    if reserve:
        seeds = torch.cat((torch.zeros_like(seeds[:, :1]), seeds), dim=1)
        gains = torch.cat((torch.zeros_like(gains[:, :1]), gains), dim=1)
    if fit_mode == "lloyd":
        return _Stage(fit_mode, whitener, None, None, seeds, None, reserve)
    # a seed represents its row at its own scale, capped
    if caps is not None:
        gains = torch.minimum(gains, caps.unsqueeze(-1))
    return _Stage(fit_mode, whitener, gains, seeds, None, caps, reserve)


@torch.no_grad()
def fit_residual_stages(
    residual: torch.Tensor,
    *,
    stages: int,
    assignment_whiteners: torch.Tensor | None,
    initial_selector_residual: torch.Tensor | None,
    sample_weights: torch.Tensor | None = None,
    kmeans_iterations: int,
    token_chunk_size: int,
    seed: int,
    fit_mode: str,
    gain_caps: torch.Tensor | None,
    reserve_zero_codeword: bool = True,
) -> tuple[torch.Tensor, list[dict[str, float | int]]]:
    """Fit ``stages`` residual stages per head (build_frozen_gsrq_multi_exit.py:400-657).

    ``residual[H,N,D]`` fp32 (D <= 128) is the raw residual at the frozen
    parent exit and is updated in place stage by stage, as the reference's
    is; with ``assignment_whiteners`` ``[H,D,D]`` (upper triangular),
    ``initial_selector_residual`` is its exact selector-space image, on
    which assignments and the gain-shape update run (a clone is updated).
    Returns fp16 tables ``[H,stages,K,D]`` on the CPU and one history dict
    per stage with the reference's keys.
    """

    if stages <= 0:
        return torch.empty(residual.shape[0], 0, CLUSTERS, residual.shape[-1], dtype=torch.float16), []
    heads, tokens, _dimension = residual.shape
    sample_weights, gain_caps = _validate(residual, sample_weights, fit_mode, assignment_whiteners,
                                          initial_selector_residual, gain_caps)
    _check_chunk(token_chunk_size)
    picks = 255 if reserve_zero_codeword else 256
    if tokens < picks:
        raise ValueError(f"fitting {CLUSTERS} codewords needs at least {picks} rows per head")
    if residual.dtype != torch.float32 or not residual.is_contiguous():
        raise ValueError("the parent residual must be contiguous fp32 [H,N,D]")
    whitener = None if assignment_whiteners is None else assignment_whiteners.to(
        device=residual.device, dtype=torch.float32).contiguous()
    selector_residual = None
    if initial_selector_residual is not None:
        selector_residual = initial_selector_residual.to(device=residual.device, dtype=torch.float32).clone()
    generator = torch.Generator(device=residual.device).manual_seed(int(seed))
    tables: list[torch.Tensor] = []
    history: list[dict[str, Any]] = []
    for stage in range(stages):
        before = float(residual.square().mean())
        working = residual if selector_residual is None else selector_residual
        book = _seed_stage(generator, working, residual, fit_mode, reserve_zero_codeword, gain_caps, whitener)
        for _ in range(kmeans_iterations):
            _raw, selector = book.deployed()
            indices = _ops.nearest_f32(working, selector)
            book.update(working, residual, indices, sample_weights)
        raw, selector = book.deployed()
        indices = _ops.nearest_f32(working, selector)
        _ops.subtract_codewords(residual, raw, indices)
        if selector_residual is not None:
            _ops.subtract_codewords(selector_residual, selector, indices)
        counts = torch.zeros((heads, raw.shape[1]), dtype=torch.int64, device=residual.device)
        counts.scatter_add_(1, indices, torch.ones_like(indices))
        tables.append(raw.half().cpu())
        history.append({
            "stage": stage,
            "residual_element_mse_before": before,
            "residual_element_mse_after": float(residual.square().mean()),
            "occupied_clusters_min": int((counts > 0).sum(dim=1).min()),
            "fit_mode": fit_mode,
            "maximum_codeword_norm": float(torch.linalg.vector_norm(raw, dim=-1).max()),
            "maximum_selector_codeword_norm": float(torch.linalg.vector_norm(selector, dim=-1).max()),
            "gain_cap_min": float(gain_caps.min()) if gain_caps is not None else -1.0,
            "gain_cap_max": float(gain_caps.max()) if gain_caps is not None else -1.0,
            "zero_codeword_reserved": int(reserve_zero_codeword),
            "zero_assignment_fraction": float(indices.eq(0).float().mean()),
            "gradient_weighted": int(sample_weights is not None),
        })
    return torch.stack(tables, dim=1), history
