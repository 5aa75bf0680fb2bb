"""CPU oracle for the offline gain-shape k-means parent fitting.

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` may import this module, as the
checker of ``jointkv_amd.gain_shape`` and of ``jkv_gain_shape_sums`` /
``jkv_subtract_codewords``; the product never calls it.

A numpy restatement, head by head, of ``fit_residual_stages``
(experiments/build_frozen_gsrq_multi_exit.py:400-657) with the seed rows
given explicitly instead of drawn from a generator:

  seeds (:478-510)   K = 255 random rows per head plus a zero codeword in
                     slot 0 (or 256 rows): unit direction and norm of each
                     working row (gskm) or the raw row (lloyd); gains capped
  deploy (:512-536)  raw = fp16(gain * shape), through W^-T when whitened
                     (W upper triangular); selector = raw W^T
  assign (:539-545)  nearest selector codeword of each working row, distance
                     (|x|^2 + |c|^2) - 2 x.c in fp32, first index on ties
  update (:546-607)  gskm: over each codeword's rows, shape = direction of
                     sum w x/max(|x|, 1e-8), gain = max(0, sum w x.shape /
                     sum w), then the cap; codeword 0 stays zero when
                     reserved; empty codewords keep their values.  lloyd:
                     plain means of the raw rows
  stage end (:610-656)  residual -= raw codeword, selector residual -=
                     selector codeword; the history record

Sums, norms and projections run in float64 (the reference's fp32 sums are
one rounding order among many); the deploy keeps the fp16 rounding and the
search keeps fp32, which decide what the fitted codec is.

Pins (tests/test_gain_shape_oracle.py): the per-codeword sums and update
against a hand-worked example; the lloyd update as the plain mean of each
codeword's rows, worked by hand; a fit of exact gain-shape data whose
codewords must come out as fp16(gain * shape) of the data; the whitened
deploy against the goal it solves for; invariants (unit shapes, gains in
[0, cap], the reserved zero codeword, non-increasing residual energy on
clustered data); ``parent_residuals`` against the greedy operator
``jointkv_oracle.hard_residual_vq_exits`` (itself pinned by an exhaustive
float64 search).  The search is the additive oracle's ``nearest``, pinned
against an exhaustive float64 search there.
"""

from __future__ import annotations

import numpy as np

from .additive_oracle import nearest

CLUSTERS = 256


def nearest_with_margin(states, table):
    """``nearest`` plus each row's gap between its best and second-best fp32
    distance relative to |x|^2 + |c_best|^2, the scale of the distance's
    rounding error (for judging which choices rounding could flip)."""

    x = np.asarray(states, dtype=np.float32)
    c = np.asarray(table, dtype=np.float32)
    xx = np.square(x).sum(axis=-1, dtype=np.float32)[:, None]
    cc = np.square(c).sum(axis=-1, dtype=np.float32)[None, :]
    dist = (xx + cc) - np.float32(2.0) * (x @ c.T).astype(np.float32)
    part = np.partition(dist, 1, axis=1)
    idx = nearest(states, table)
    scale = xx[:, 0].astype(np.float64) + cc[0, idx].astype(np.float64) + 1e-30
    return idx, (part[:, 1] - part[:, 0]).astype(np.float64) / scale


def codeword_sums(rows, idx, clusters, weights=None):
    """Per-codeword sums of one head, float64: (unit-direction sums, row sums,
    weight sums, sums of |w x| for tolerances).  rows [N,D], idx [N]."""

    x = np.asarray(rows, dtype=np.float64)
    idx = np.asarray(idx, dtype=np.int64)
    w = np.ones(len(x)) if weights is None else np.asarray(weights, dtype=np.float64)
    norm = np.maximum(np.sqrt(np.square(x).sum(axis=1)), 1e-8)
    unit = x / norm[:, None] * w[:, None]
    wx = x * w[:, None]
    d = x.shape[1]
    shape_sums = np.zeros((clusters, d))
    raw_sums = np.zeros((clusters, d))
    abs_sums = np.zeros((clusters, d))
    den = np.zeros(clusters)
    keep = (idx >= 0) & (idx < clusters)
    np.add.at(shape_sums, idx[keep], unit[keep])
    np.add.at(raw_sums, idx[keep], wx[keep])
    np.add.at(abs_sums, idx[keep], np.abs(wx[keep]))
    np.add.at(den, idx[keep], w[keep])
    return shape_sums, raw_sums, den, abs_sums


def gskm_update(shapes, gains, shape_sums, raw_sums, den, cap=None, reserve=True):
    """One gain-shape update of one head from its sums (float64)."""

    shapes = np.array(shapes, dtype=np.float64)
    gains = np.array(gains, dtype=np.float64)
    length = np.sqrt(np.square(shape_sums).sum(axis=1))
    ok = (den > 0) & (length > 1e-8)
    if reserve:
        ok[0] = False
    shapes[ok] = shape_sums[ok] / length[ok, None]
    gains[ok] = np.maximum((raw_sums[ok] * shapes[ok]).sum(axis=1) / den[ok], 0.0)
    if cap is not None:
        gains = np.minimum(gains, cap)
    if reserve:
        shapes[0] = 0.0
        gains[0] = 0.0
    return shapes, gains


def deploy(shapes, gains, means, whitener, fit_mode):
    """fp16-rounded raw codewords (float32) and their selector images."""

    if fit_mode == "gskm":
        goal = np.asarray(gains, dtype=np.float64)[:, None] * np.asarray(shapes, dtype=np.float64)
        if whitener is None:
            raw = goal
        else:
            # W raw^T = goal^T over W's upper triangle (a triangular solve
            # reads nothing else)
            raw = np.linalg.solve(np.triu(np.asarray(whitener, dtype=np.float64)), goal.T).T
    else:
        raw = np.asarray(means, dtype=np.float64)
    raw = raw.astype(np.float32).astype(np.float16).astype(np.float32)
    if whitener is None:
        return raw, raw
    return raw, (raw.astype(np.float64) @ np.asarray(whitener, dtype=np.float64).T).astype(np.float32)


def fit_residual_stages(residual, seed_rows, *, stages, whitener=None, selector_residual=None, weights=None,
                        iterations, fit_mode="gskm", caps=None, reserve=True, forced_tables=None):
    """residual [H,N,D] (a copy is updated), seed_rows[stage][head] the rows
    chosen as that head's seeds.  Returns (tables fp16 [H,stages,K,D],
    history, smallest relative search margin met).

    ``forced_tables`` [H,stages,K,D] (fp16 values): each stage still fits its
    own table (returned), but ends with the given one: the residual update
    and the history use it, so that the next stage starts from the residual
    those codewords leave (a run under test hands its own tables in)."""

    res = np.array(residual, dtype=np.float32)
    sel = None if selector_residual is None else np.array(selector_residual, dtype=np.float32)
    heads = res.shape[0]
    tables, history = [], []
    smallest = np.inf
    for stage in range(stages):
        before = float(np.square(res.astype(np.float64)).mean())
        work = res if sel is None else sel
        books = []
        for h in range(heads):
            rows = np.asarray(seed_rows[stage][h], dtype=np.int64)
            picked = work[h][rows].astype(np.float64)
            g = np.sqrt(np.square(picked).sum(axis=1))
            s = picked / np.maximum(g, 1e-8)[:, None] if fit_mode == "gskm" else res[h][rows].astype(np.float64)
            if reserve:
                s = np.concatenate([np.zeros((1, s.shape[1])), s])
                g = np.concatenate([[0.0], g])
            if caps is not None:
                g = np.minimum(g, caps[h])
            books.append([s, g])
        w_h = [None if weights is None else np.asarray(weights[h]) for h in range(heads)]
        for _ in range(iterations):
            for h in range(heads):
                s, g = books[h]
                W = None if whitener is None else whitener[h]
                raw, selc = deploy(s, g, s, W, fit_mode)
                idx, gap = nearest_with_margin(work[h], selc)
                smallest = min(smallest, float(gap.min()))
                if fit_mode == "gskm":
                    ssum, rsum, den, _abs = codeword_sums(work[h], idx, len(s), w_h[h])
                    books[h] = list(gskm_update(s, g, ssum, rsum, den, None if caps is None else caps[h], reserve))
                else:
                    _ss, rsum, den, _abs = codeword_sums(res[h], idx, len(s))
                    ok = den > 0
                    if reserve:
                        ok[0] = False
                    s = np.array(s)
                    s[ok] = rsum[ok] / den[ok, None]
                    if reserve:
                        s[0] = 0.0
                    books[h] = [s, g]
        raws, sels, idxs = [], [], []
        own = []
        for h in range(heads):
            s, g = books[h]
            W = None if whitener is None else whitener[h]
            raw, selc = deploy(s, g, s, W, fit_mode)
            own.append(raw)
            if forced_tables is not None:
                raw = np.asarray(forced_tables[h, stage], dtype=np.float32)
                if W is not None:
                    selc = (raw.astype(np.float64) @ np.asarray(W, dtype=np.float64).T).astype(np.float32)
                else:
                    selc = raw
            idx, gap = nearest_with_margin(work[h], selc)
            smallest = min(smallest, float(gap.min()))
            res[h] -= raw[idx]
            if sel is not None:
                sel[h] -= selc[idx]
            raws.append(raw)
            sels.append(selc)
            idxs.append(idx)
        raws, sels, idxs = np.stack(raws), np.stack(sels), np.stack(idxs)
        tables.append(np.stack(own).astype(np.float16))
        history.append({
            "stage": stage,
            "residual_element_mse_before": before,
            "residual_element_mse_after": float(np.square(res.astype(np.float64)).mean()),
            "occupied_clusters_min": int(min(len(np.unique(i)) for i in idxs)),
            "fit_mode": fit_mode,
            "maximum_codeword_norm": float(np.sqrt(np.square(raws.astype(np.float64)).sum(-1)).max()),
            "maximum_selector_codeword_norm": float(np.sqrt(np.square(sels.astype(np.float64)).sum(-1)).max()),
            "gain_cap_min": float(np.min(caps)) if caps is not None else -1.0,
            "gain_cap_max": float(np.max(caps)) if caps is not None else -1.0,
            "zero_codeword_reserved": int(reserve),
            "zero_assignment_fraction": float((idxs == 0).mean()),
            "gradient_weighted": int(weights is not None),
        })
    return np.stack(tables, axis=1), history, smallest


def parent_residuals(states, tables, whitener, depth):
    """The frozen parent's residuals at exit ``depth``
    (build_frozen_gsrq_multi_exit.py:661-738): states [B,H,T,D], tables
    [H,S,K,D] (deployed values), whitener [H,D,D] or None.  Returns (raw
    residual [H,B*T,D] fp32, selector residual or None, reconstruction
    [B,H,T,D] fp32, smallest relative search margin)."""

    x = np.asarray(states, dtype=np.float32)
    batch, heads, tokens, dim = x.shape
    raw = np.ascontiguousarray(x.transpose(1, 0, 2, 3).reshape(heads, batch * tokens, dim))
    decoded = np.zeros_like(raw)
    tabs = np.asarray(tables, dtype=np.float32)[:, :depth]
    sel = sel_tabs = None
    if whitener is not None:
        w = np.asarray(whitener, dtype=np.float64)
        sel = np.einsum("hde,hne->hnd", w, raw.astype(np.float64)).astype(np.float32)
        sel_tabs = np.einsum("hske,hde->hskd", tabs.astype(np.float64), w).astype(np.float32)
    smallest = np.inf
    for stage in range(depth):
        for h in range(heads):
            search = raw[h] if sel is None else sel[h]
            table = tabs[h, stage] if sel is None else sel_tabs[h, stage]
            idx, gap = nearest_with_margin(search, table)
            smallest = min(smallest, float(gap.min()))
            decoded[h] += tabs[h, stage][idx]
            raw[h] -= tabs[h, stage][idx]
            if sel is not None:
                sel[h] -= sel_tabs[h, stage][idx]
    recon = decoded.reshape(heads, batch, tokens, dim).transpose(1, 0, 2, 3)
    return raw, sel, recon, smallest
