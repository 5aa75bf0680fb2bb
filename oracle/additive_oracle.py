"""CPU oracle for the offline multi-exit additive coordinate refinement.

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` may import this module, as the
checker of ``jointkv_amd.additive_refinement`` and of ``jkv_nearest_f32``;
the product never calls it.

A numpy float32 restatement, head by head and row by row, of
src/jointkv/nested_vq.py: ``_nearest_indices`` without whiteners (:178-215:
distance (|x|^2 + |c|^2) - 2 x.c in fp32, first index on ties) and the
reverse coordinate sweep of ``multi_exit_additive_coordinate_refinement``
(:583-741: per stage, target = old word + sum_m w_m (x - recon_m) / sum_m w_m
over the exits m > stage with w_m > 0, then nearest, then every affected
exit's reconstruction moves by new word - old word).

It also restates ``_nearest_topk_indices`` (:218-260) and the sliding
two-stage block sweep of ``multi_exit_additive_block_refinement``
(:757-1001), row by row.

Pins (tests/test_additive_refinement.py): every stage's choice in a
coordinate sweep is checked against an exhaustive float64 search of the
weighted multi-exit objective over all K candidates (others fixed as the
sweep has left them); a block sweep whose shortlist holds every codeword is
checked against an exhaustive float64 search over all K^2 pairs; top-k
against a float64 sort; and neither sweep ever raises the weighted
objective.
"""

from __future__ import annotations

import numpy as np


def nearest(states, table):
    """states [N,D], table [K,D] float32 -> int64 [N] (nested_vq.py:203-214)."""

    x = np.asarray(states, dtype=np.float32)
    c = np.asarray(table, dtype=np.float32)
    xx = np.square(x).sum(axis=-1, dtype=np.float32)[:, None]
    cc = np.square(c).sum(axis=-1, dtype=np.float32)[None, :]
    dist = (xx + cc) - np.float32(2.0) * (x @ c.T).astype(np.float32)
    return dist.argmin(axis=-1).astype(np.int64)


def coordinate_refinement(states, stage_tables, initial_indices, prefixes, exit_weights, sweeps=1):
    """states [B,H,T,D]; stage_tables list of [H,K,D]; initial_indices
    [B,H,T,S].  Returns (recon {prefix: float32 [B,H,T,D]}, int64 indices
    [B,H,T,S], weighted objective after each sweep, initial objective)."""

    x4 = np.asarray(states, dtype=np.float32)
    batch, heads, tokens, dim = x4.shape
    req = sorted({int(p) for p in prefixes})
    w = [float(v) for v in exit_weights]
    depth = req[-1]
    tabs = [np.asarray(t, dtype=np.float32) for t in stage_tables[:depth]]
    x = x4.transpose(1, 0, 2, 3).reshape(heads, batch * tokens, dim)
    idx = np.asarray(initial_indices).transpose(1, 0, 2, 3).reshape(heads, batch * tokens, depth).astype(np.int64)
    recon = {}
    for h in range(heads):
        run = np.zeros((batch * tokens, dim), dtype=np.float32)
        for s in range(depth):
            run = run + tabs[s][h][idx[h, :, s]]
            if s + 1 in req:
                recon.setdefault(s + 1, np.zeros_like(x))[h] = run

    def objective():
        mse = [float(np.square(x - recon[p]).mean(dtype=np.float64)) for p in req]
        return sum(wi * m for wi, m in zip(w, mse)) / sum(w)

    initial = objective()
    history = []
    for _sweep in range(sweeps):
        for s in range(depth - 1, -1, -1):
            aff = [(p, wi) for p, wi in zip(req, w) if p > s and wi > 0]
            wsum = sum(wi for _p, wi in aff)
            for h in range(heads):
                old = tabs[s][h][idx[h, :, s]]
                resid = np.zeros_like(old)
                for p, wi in aff:
                    resid = resid + np.float32(wi) * (x[h] - recon[p][h])
                target = old + resid * np.float32(1.0 / wsum)
                new = nearest(target, tabs[s][h])
                delta = tabs[s][h][new] - old
                for p, _wi in aff:
                    recon[p][h] = recon[p][h] + delta
                idx[h, :, s] = new
        history.append(objective())
    out = {p: r.reshape(heads, batch, tokens, dim).transpose(1, 0, 2, 3) for p, r in recon.items()}
    return out, idx.reshape(heads, batch, tokens, depth).transpose(1, 0, 2, 3), history, initial


def nearest_topk(states, table, m, excluded=None):
    """The m nearest rows of table per state, nearest first, ties in index
    order, one index per row left out (nested_vq.py:218-260)."""

    x = np.asarray(states, dtype=np.float32)
    c = np.asarray(table, dtype=np.float32)
    xx = np.square(x).sum(axis=-1, dtype=np.float32)[:, None]
    cc = np.square(c).sum(axis=-1, dtype=np.float32)[None, :]
    dist = (xx + cc) - np.float32(2.0) * (x @ c.T).astype(np.float32)
    if excluded is not None:
        dist[np.arange(len(x)), np.asarray(excluded)] = np.inf
    return np.argsort(dist, axis=-1, kind="stable")[:, :m].astype(np.int64)


def block_refinement(states, stage_tables, initial_indices, prefixes, exit_weights, sweeps=1, shortlist=4):
    """The sliding-pair block sweep of nested_vq.py:838-958, row by row in
    numpy float32.  Returns (recon {prefix: [B,H,T,D]}, indices [B,H,T,S],
    weighted objective after each sweep, initial objective)."""

    x4 = np.asarray(states, dtype=np.float32)
    batch, heads, tokens, dim = x4.shape
    req = sorted({int(p) for p in prefixes})
    w = [float(v) for v in exit_weights]
    depth = req[-1]
    tabs = [np.asarray(t, dtype=np.float32) for t in stage_tables[:depth]]
    x = x4.transpose(1, 0, 2, 3).reshape(heads, batch * tokens, dim)
    idx = np.asarray(initial_indices).transpose(1, 0, 2, 3).reshape(heads, batch * tokens, depth).astype(np.int64)
    recon = {}
    for h in range(heads):
        run = np.zeros((batch * tokens, dim), dtype=np.float32)
        for s in range(depth):
            run = run + tabs[s][h][idx[h, :, s]]
            if s + 1 in req:
                recon.setdefault(s + 1, np.zeros_like(x))[h] = run

    def objective():
        mse = [float(np.square(x - recon[p]).mean(dtype=np.float64)) for p in req]
        return sum(wi * m for wi, m in zip(w, mse)) / sum(w)

    initial = objective()
    history = []
    for _sweep in range(sweeps):
        for first in range(depth - 2, -1, -1):
            pair = (first, first + 1)
            aff = [(p, wi) for p, wi in zip(req, w) if p > first and wi > 0]
            for h in range(heads):
                for n in range(batch * tokens):
                    olds = [idx[h, n, s] for s in pair]
                    ow = [tabs[s][h][o] for s, o in zip(pair, olds)]
                    lists = []
                    for s, o, word in zip(pair, olds, ow):
                        local = [(p, wi) for p, wi in aff if p > s]
                        wsum = sum(wi for _p, wi in local)
                        resid = np.zeros(dim, dtype=np.float32)
                        for p, wi in local:
                            resid = resid + np.float32(wi) * (x[h, n] - recon[p][h, n])
                        target = word + resid / np.float32(wsum)
                        alt = nearest_topk(target[None], tabs[s][h], shortlist - 1, [o])[0]
                        lists.append([o] + list(alt))
                    best, choice = np.inf, (0, 0)
                    for a in range(shortlist):
                        for b in range(shortlist):
                            cost = np.float32(0.0)
                            for p, wi in aff:
                                base = x[h, n] - recon[p][h, n] + ow[0]
                                cand = tabs[pair[0]][h][lists[0][a]]
                                if p > pair[1]:
                                    base = base + ow[1]
                                    cand = cand + tabs[pair[1]][h][lists[1][b]]
                                cost = cost + np.float32(wi) * np.square(base - cand).sum(dtype=np.float32)
                            if cost < best:
                                best, choice = cost, (a, b)
                    news = [lists[0][choice[0]], lists[1][choice[1]]]
                    for k, s in enumerate(pair):
                        delta = tabs[s][h][news[k]] - ow[k]
                        for p, _wi in aff:
                            if p > s:
                                recon[p][h, n] = recon[p][h, n] + delta
                        idx[h, n, s] = news[k]
        history.append(objective())
    out = {p: r.reshape(heads, batch, tokens, dim).transpose(1, 0, 2, 3) for p, r in recon.items()}
    return out, idx.reshape(heads, batch, tokens, depth).transpose(1, 0, 2, 3), history, initial
