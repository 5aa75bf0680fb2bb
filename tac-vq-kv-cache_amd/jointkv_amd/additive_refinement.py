"""Offline multi-exit additive coordinate refinement on the MI355X
(src/jointkv/nested_vq.py:582-741, ``multi_exit_additive_coordinate_refinement``).

Given greedy residual indices, a reverse sweep re-chooses one stage at a
time with the others fixed.  For stage ``s`` the exits ``m`` that include it
share one Euclidean target, ``old_word + sum_m w_m (x - recon_m) / sum_m w_m``,
so the stage's new index is that target's nearest codeword and every step is
non-increasing for the weighted multi-exit objective (nested_vq.py:596-604).

The search is ``jkv_nearest_f32`` (fp32 tables, as the reference keeps them
for this encoder, nested_vq.py:636-639); the target and reconstruction
updates are elementwise tensor arithmetic in the reference's order.  Index
layout and decoder are unchanged: the output indices decode with the same
tables as the greedy ones.
"""

from __future__ import annotations

import math
from typing import Iterable, Sequence

import torch

from . import _ops


def _gather_words(table: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """``[H,N]`` indices of one ``[H,K,D]`` table -> ``[H,N,D]`` (nested_vq.py:568-580)."""

    return torch.gather(table, 1, indices.unsqueeze(-1).expand(-1, -1, table.shape[-1]))


@torch.no_grad()
def multi_exit_additive_coordinate_refinement(
    states: torch.Tensor,
    stage_tables: Sequence[torch.Tensor],
    initial_indices: torch.Tensor,
    *,
    prefixes: Iterable[int],
    exit_weights: Sequence[float],
    sweeps: int = 1,
    token_chunk_size: int = 4096,
):
    """Refine ``initial_indices`` ``[B,H,T,S]`` of ``states`` ``[B,H,T,D]``
    against the exits in ``prefixes`` jointly.  Returns
    ``({prefix: reconstruction [B,H,T,D] in states' dtype}, uint8 indices
    [B,H,T,S], diagnostics)`` with the reference's diagnostics keys
    (nested_vq.py:727-741).  ``token_chunk_size`` is validated as the
    reference does; the HIP search needs no chunking."""

    requested = tuple(sorted({int(prefix) for prefix in prefixes}))
    weights = tuple(float(weight) for weight in exit_weights)
    if states.ndim != 4 or not torch.isfinite(states).all():
        raise ValueError("states must have finite [B,H,T,D] layout")
    if not requested or requested[0] <= 0 or requested[-1] > len(stage_tables):
        raise ValueError("prefixes must lie inside the materialized stages")
    if len(weights) != len(requested) or any(not math.isfinite(w) or w < 0 for w in weights):
        raise ValueError("one finite non-negative weight is required per exit")
    if not any(w > 0 for w in weights):
        raise ValueError("at least one exit weight must be positive")
    if sweeps <= 0 or token_chunk_size <= 0:
        raise ValueError("coordinate sweeps and token chunks must be positive")
    batch, heads, tokens, dim = map(int, states.shape)
    depth = requested[-1]
    if tuple(initial_indices.shape) != (batch, heads, tokens, depth):
        raise ValueError("initial indices differ from the requested stage geometry")
    tables = [t.to(device=states.device, dtype=torch.float32).contiguous() for t in stage_tables[:depth]]
    for stage, table in enumerate(tables):
        if table.ndim != 3 or table.shape[0] != heads or table.shape[2] != dim:
            raise ValueError(f"stage {stage} table geometry differs from states")
        if not torch.isfinite(table).all():
            raise ValueError(f"stage {stage} table is non-finite")

    x = states.permute(1, 0, 2, 3).reshape(heads, batch * tokens, dim).float()
    idx = initial_indices.permute(1, 0, 2, 3).reshape(heads, batch * tokens, depth).long().clone()
    recon: dict[int, torch.Tensor] = {}
    running = torch.zeros_like(x)
    for stage, table in enumerate(tables):
        col = idx[..., stage]
        if int(col.min()) < 0 or int(col.max()) >= table.shape[1]:
            raise ValueError(f"stage {stage} index is outside its codebook")
        running.add_(_gather_words(table, col))
        if stage + 1 in requested:
            recon[stage + 1] = running.clone()

    def objective():
        per_exit = {str(p): float((x - recon[p]).square().mean().item()) for p in requested}
        weighted = sum(w * per_exit[str(p)] for p, w in zip(requested, weights)) / sum(weights)
        return weighted, per_exit

    initial_objective, initial_per_exit = objective()
    history = []
    for sweep in range(sweeps):
        changed: dict[str, float] = {}
        for stage in range(depth - 1, -1, -1):
            affected = [(p, w) for p, w in zip(requested, weights) if p > stage and w > 0]
            weight_sum = sum(w for _p, w in affected)
            if weight_sum <= 0:
                raise ValueError(f"stage {stage} is not covered by a positive exit")
            table = tables[stage]
            old = idx[..., stage]
            old_words = _gather_words(table, old)
            target = old_words.clone()
            residual = torch.zeros_like(target)
            for p, w in affected:
                residual.add_(x - recon[p], alpha=w)
            target.add_(residual, alpha=1.0 / weight_sum)
            new = _ops.nearest_f32(target, table)
            changed[str(stage + 1)] = float(new.ne(old).float().mean().item())
            delta = _gather_words(table, new) - old_words
            for p, _w in affected:
                recon[p].add_(delta)
            idx[..., stage] = new
        weighted, per_exit = objective()
        history.append({
            "sweep": sweep + 1,
            "weighted_objective": weighted,
            "per_exit_mse": per_exit,
            "changed_fraction_by_stage": changed,
            "mean_changed_fraction": sum(changed.values()) / len(changed),
        })
    final_objective, final_per_exit = objective()
    outputs = {
        p: r.reshape(heads, batch, tokens, dim).permute(1, 0, 2, 3).to(dtype=states.dtype).contiguous()
        for p, r in recon.items()
    }
    refined = idx.reshape(heads, batch, tokens, depth).permute(1, 0, 2, 3).to(torch.uint8).contiguous()
    diagnostics = {
        "mode": "multi_exit_additive_coordinate",
        "coordinate_order": "reverse",
        "sweeps": sweeps,
        "prefixes": list(requested),
        "exit_weights": list(weights),
        "initial_weighted_objective": initial_objective,
        "final_weighted_objective": final_objective,
        "relative_objective_change": final_objective / max(initial_objective, 1e-30) - 1.0,
        "initial_per_exit_mse": initial_per_exit,
        "final_per_exit_mse": final_per_exit,
        "sweep_history": history,
    }
    return outputs, refined, diagnostics


@torch.no_grad()
def multi_exit_additive_block_refinement(
    states: torch.Tensor,
    stage_tables: Sequence[torch.Tensor],
    initial_indices: torch.Tensor,
    *,
    prefixes: Iterable[int],
    exit_weights: Sequence[float],
    sweeps: int = 1,
    shortlist_size: int = 4,
    token_chunk_size: int = 512,
):
    """Sliding two-stage block refinement (nested_vq.py:757-1001).

    Each reverse sweep visits the stage pairs ``(S-1,S), ..., (1,2)``.  Per
    pair, each stage's shortlist is its old index followed by the
    ``shortlist_size - 1`` nearest other codewords of its coordinate target
    (``jkv_nearest_topk_f32``); the ``shortlist_size^2`` products are scored
    with the exact weighted error of every affected exit and the lowest wins,
    the old pair first on ties.  Rows are independent, so the row chunks
    only bound the ``[H,n,L,L,D]`` fp32 score temporaries: at least
    ``token_chunk_size`` rows are scored at a time, and more while those
    temporaries stay within 512 MiB (the reference's 512-row default would
    otherwise leave the sweep bound by per-chunk launch overhead)."""

    requested = tuple(sorted({int(prefix) for prefix in prefixes}))
    weights = tuple(float(weight) for weight in exit_weights)
    if states.ndim != 4 or not torch.isfinite(states).all():
        raise ValueError("states must have finite [B,H,T,D] layout")
    if not requested or requested[0] <= 0 or requested[-1] > len(stage_tables):
        raise ValueError("prefixes must lie inside the materialized stages")
    if len(weights) != len(requested) or any(not math.isfinite(w) or w < 0 for w in weights):
        raise ValueError("one finite non-negative weight is required per exit")
    if not any(w > 0 for w in weights):
        raise ValueError("at least one exit weight must be positive")
    if sweeps <= 0 or shortlist_size < 2 or token_chunk_size <= 0:
        raise ValueError("invalid block-refinement search geometry")
    batch, heads, tokens, dim = map(int, states.shape)
    depth = requested[-1]
    if depth < 2:
        raise ValueError("two-stage refinement requires at least two stages")
    if tuple(initial_indices.shape) != (batch, heads, tokens, depth):
        raise ValueError("initial indices differ from the requested stage geometry")
    tables = [t.to(device=states.device, dtype=torch.float32).contiguous() for t in stage_tables[:depth]]
    for stage, table in enumerate(tables):
        if table.ndim != 3 or table.shape[0] != heads or table.shape[2] != dim:
            raise ValueError(f"stage {stage} table geometry differs from states")
        if table.shape[1] < shortlist_size or not torch.isfinite(table).all():
            raise ValueError(f"stage {stage} cannot support the requested shortlist")
    if shortlist_size - 1 > 8:
        raise ValueError("the HIP shortlist search takes at most 8 alternatives (shortlist_size <= 9)")

    x = states.permute(1, 0, 2, 3).reshape(heads, batch * tokens, dim).float()
    idx = initial_indices.permute(1, 0, 2, 3).reshape(heads, batch * tokens, depth).long().clone()
    recon: dict[int, torch.Tensor] = {}
    running = torch.zeros_like(x)
    for stage, table in enumerate(tables):
        col = idx[..., stage]
        if int(col.min()) < 0 or int(col.max()) >= table.shape[1]:
            raise ValueError(f"stage {stage} index is outside its codebook")
        running.add_(_gather_words(table, col))
        if stage + 1 in requested:
            recon[stage + 1] = running.clone()

    def objective():
        per_exit = {str(p): float((x - recon[p]).square().mean().item()) for p in requested}
        weighted = sum(w * per_exit[str(p)] for p, w in zip(requested, weights)) / sum(weights)
        return weighted, per_exit

    def candidate_words(table, shortlist):
        flat = shortlist.reshape(heads, -1)
        return _gather_words(table, flat).reshape(*shortlist.shape, dim)

    initial_objective, initial_per_exit = objective()
    history = []
    total = x.shape[1]
    L = shortlist_size
    rows_per_chunk = max(token_chunk_size, (512 << 20) // (4 * heads * L * L * dim))
    for sweep in range(sweeps):
        blocks = []
        for first in range(depth - 2, -1, -1):
            pair = (first, first + 1)
            affected = [(p, w) for p, w in zip(requested, weights) if p > first and w > 0]
            changed = [0, 0]
            for start in range(0, total, rows_per_chunk):
                stop = min(total, start + rows_per_chunk)
                xc = x[:, start:stop]
                olds = [idx[:, start:stop, s] for s in pair]
                old_words = [_gather_words(tables[s], o) for s, o in zip(pair, olds)]
                shortlists, cands = [], []
                for s, o, ow in zip(pair, olds, old_words):
                    local = [(p, w) for p, w in affected if p > s]
                    wsum = sum(w for _p, w in local)
                    if wsum <= 0:
                        raise ValueError(f"stage {s} lacks a positive exit")
                    residual = torch.zeros_like(ow)
                    for p, w in local:
                        residual.add_(xc - recon[p][:, start:stop], alpha=w)
                    target = ow + residual / wsum
                    alt = _ops.nearest_topk_f32(target, tables[s], L - 1, excluded=o)
                    sl = torch.cat((o.unsqueeze(-1), alt), dim=-1)
                    shortlists.append(sl)
                    cands.append(candidate_words(tables[s], sl))
                cost = torch.zeros((heads, stop - start, L, L), dtype=torch.float32, device=x.device)
                for p, w in affected:
                    base = xc - recon[p][:, start:stop] + old_words[0]
                    if p > pair[1]:
                        base = base + old_words[1]
                        csum = cands[0].unsqueeze(-2) + cands[1].unsqueeze(-3)
                    else:
                        csum = cands[0].unsqueeze(-2)
                    cost.add_((base.unsqueeze(-2).unsqueeze(-2) - csum).square().sum(dim=-1), alpha=w)
                choice = cost.flatten(-2).argmin(dim=-1)
                news = [torch.gather(shortlists[0], -1, (choice // L).unsqueeze(-1)).squeeze(-1),
                        torch.gather(shortlists[1], -1, (choice % L).unsqueeze(-1)).squeeze(-1)]
                for k in range(2):
                    changed[k] += int(news[k].ne(olds[k]).sum())
                deltas = [_gather_words(tables[s], n) - ow for s, n, ow in zip(pair, news, old_words)]
                for p, _w in affected:
                    for s, dlt in zip(pair, deltas):
                        if p > s:
                            recon[p][:, start:stop].add_(dlt)
                for s, n in zip(pair, news):
                    idx[:, start:stop, s] = n
            blocks.append({"stages": [first + 1, first + 2],
                           "changed_fraction": [changed[0] / (heads * total), changed[1] / (heads * total)]})
        weighted, per_exit = objective()
        history.append({
            "sweep": sweep + 1,
            "weighted_objective": weighted,
            "per_exit_mse": per_exit,
            "blocks": blocks,
            "mean_block_changed_fraction": sum(sum(b["changed_fraction"]) / 2 for b in blocks) / len(blocks),
        })
    final_objective, final_per_exit = objective()
    outputs = {
        p: r.reshape(heads, batch, tokens, dim).permute(1, 0, 2, 3).to(dtype=states.dtype).contiguous()
        for p, r in recon.items()
    }
    refined = idx.reshape(heads, batch, tokens, depth).permute(1, 0, 2, 3).to(torch.uint8).contiguous()
    diagnostics = {
        "mode": "multi_exit_additive_block",
        "block_schedule": "reverse_sliding_pairs",
        "sweeps": sweeps,
        "shortlist_size": shortlist_size,
        "prefixes": list(requested),
        "exit_weights": list(weights),
        "initial_weighted_objective": initial_objective,
        "final_weighted_objective": final_objective,
        "relative_objective_change": final_objective / max(initial_objective, 1e-30) - 1.0,
        "initial_per_exit_mse": initial_per_exit,
        "final_per_exit_mse": final_per_exit,
        "sweep_history": history,
    }
    return outputs, refined, diagnostics
