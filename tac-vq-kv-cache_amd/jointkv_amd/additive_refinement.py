"""Offline multi-exit additive refinement of residual-VQ indices on the MI355X.

Drop-in for the two offline encoders of src/jointkv/nested_vq.py,
``multi_exit_additive_coordinate_refinement`` (:583-741) and
``multi_exit_additive_block_refinement`` (:757-1001): same arguments, error
texts, outputs and diagnostics keys.  Both start from greedy indices and
re-choose stages in reverse so that the weighted objective
``sum_p w_p mean|x - recon_p|^2 / sum_p w_p`` over the requested exits never
rises.

Design.  The working state is one stacked tensor of exit reconstructions
``R`` (``[exits, H, N, D]`` fp32, slice e for the e-th requested prefix):

* a stage's coordinate target is its current word plus the weight-averaged
  error ``x - R[e]`` of the weighted exits containing it, one ``tensordot``
  over the stack;
* moving a stage from word ``a`` to ``b`` adds ``b - a`` to those exits in one
  ``index_add_`` (the same fp32 additions, in the same order, as the
  reference's per-exit updates, so equal decisions give equal bits);
* the objective is read off ``x - R``.

The nearest and top-k searches are ``jkv_nearest_f32`` and
``jkv_nearest_topk_f32``.  A whole block step (scoring the ``L x L``
shortlist pairs of two stages against every weighted exit, choosing, and
updating the reconstructions) is one ``jkv_pair_block_select`` launch, one wave
per row, with no per-candidate temporaries; ``token_chunk_size`` is
therefore validated but bounds nothing.

Only weighted exits move (as in the reference): an exit of weight 0 keeps
the reconstruction of the initial indices.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Iterable, Sequence

import torch

from . import _lib, _ops


def _checked_exits(stage_tables, prefixes, exit_weights) -> tuple[tuple[int, ...], tuple[float, ...]]:
    prefixes = tuple(sorted({int(p) for p in prefixes}))
    weights = tuple(float(w) for w in exit_weights)
    if not prefixes or prefixes[0] <= 0 or prefixes[-1] > len(stage_tables):
        raise ValueError("prefixes must lie inside the materialized stages")
    if len(weights) != len(prefixes) or any(not math.isfinite(w) or w < 0 for w in weights):
        raise ValueError("one finite non-negative weight is required per exit")
    if not any(w > 0 for w in weights):
        raise ValueError("at least one exit weight must be positive")
    return prefixes, weights


@dataclass
class _Sweep:
    """Flattened problem: rows ``[H, N=B*T]``, fp32 tables, int64 indices
    ``[H, N, S]`` and the stack of exit reconstructions."""

    shape: tuple[int, int, int, int]  # B, H, T, D of the states
    dtype: torch.dtype
    x: torch.Tensor
    tables: list[torch.Tensor]
    idx: torch.Tensor
    prefixes: tuple[int, ...]
    weights: tuple[float, ...]
    recon: torch.Tensor

    @classmethod
    def build(cls, states, stage_tables, initial_indices, prefixes, weights, depth_check=None, table_check=None):
        batch, heads, tokens, dim = map(int, states.shape)
        depth = prefixes[-1]
        if depth_check is not None:
            depth_check(depth)
        if tuple(initial_indices.shape) != (batch, heads, tokens, depth):
            raise ValueError("initial indices differ from the requested stage geometry")
        tables = []
        for stage, table in enumerate(stage_tables[:depth]):
            table = table.to(device=states.device, dtype=torch.float32).contiguous()
            if table.ndim != 3 or table.shape[0] != heads or table.shape[2] != dim:
                raise ValueError(f"stage {stage} table geometry differs from states")
            if table_check is not None:
                table_check(stage, table)
            elif not torch.isfinite(table).all():
                raise ValueError(f"stage {stage} table is non-finite")
            tables.append(table)
        rows = batch * tokens
        x = states.detach().float().permute(1, 0, 2, 3).reshape(heads, rows, dim).contiguous()
        # a private copy: the sweeps write indices in place, and for B = 1 the
        # permuted view would still alias the caller's tensor
        idx = initial_indices.detach().long().permute(1, 0, 2, 3).reshape(heads, rows, depth).clone(
            memory_format=torch.contiguous_format)
        for stage, table in enumerate(tables):
            lo, hi = torch.aminmax(idx[..., stage])
            if int(lo) < 0 or int(hi) >= table.shape[1]:
                raise ValueError(f"stage {stage} index is outside its codebook")
        sweep = cls((batch, heads, tokens, dim), states.dtype, x, tables, idx, prefixes, weights, torch.empty(0))
        sweep.recon = sweep.decode(idx)
        return sweep

    def word(self, stage: int, indices: torch.Tensor) -> torch.Tensor:
        """``[H, N]`` indices of one stage -> ``[H, N, D]`` codewords."""

        table = self.tables[stage]
        return torch.gather(table, 1, indices.unsqueeze(-1).expand(-1, -1, table.shape[-1]))

    def decode(self, idx: torch.Tensor) -> torch.Tensor:
        """Reconstruction at every requested exit, ``[exits, H, N, D]``:
        the running fp32 sum of the stages' words in stage order."""

        out = torch.empty((len(self.prefixes), *self.x.shape), dtype=torch.float32, device=self.x.device)
        running = torch.zeros_like(self.x)
        e = 0
        for stage in range(self.prefixes[-1]):
            running += self.word(stage, idx[..., stage])
            if stage + 1 == self.prefixes[e]:
                out[e] = running
                e += 1
        return out

    def members(self, stage: int) -> list[int]:
        """Stack slots of the weighted exits that contain ``stage``."""

        return [e for e, (p, w) in enumerate(zip(self.prefixes, self.weights)) if p > stage and w > 0]

    def weight_sum(self, slots: Sequence[int]) -> float:
        return sum(self.weights[e] for e in slots)

    def target(self, stage: int, slots: Sequence[int], current: torch.Tensor) -> torch.Tensor:
        """The stage's exact coordinate target: its current words plus the
        weight-averaged error of the exits in ``slots``."""

        w = torch.tensor([self.weights[e] for e in slots], dtype=torch.float32, device=self.x.device)
        index = torch.tensor(list(slots), dtype=torch.long, device=self.x.device)
        error = self.x.unsqueeze(0) - self.recon.index_select(0, index)
        return self.word(stage, current) + torch.tensordot(w, error, dims=1) / self.weight_sum(slots)

    def move(self, slots: Sequence[int], change: torch.Tensor) -> None:
        index = torch.tensor(list(slots), dtype=torch.long, device=self.x.device)
        self.recon.index_add_(0, index, change.unsqueeze(0).expand(len(slots), -1, -1, -1))

    def objective(self) -> tuple[float, dict[str, float]]:
        mse = (self.x.unsqueeze(0) - self.recon).square().mean(dim=(1, 2, 3)).tolist()
        per_exit = {str(p): float(v) for p, v in zip(self.prefixes, mse)}
        weighted = sum(w * m for w, m in zip(self.weights, mse)) / sum(self.weights)
        return weighted, per_exit

    def results(self) -> tuple[dict[int, torch.Tensor], torch.Tensor]:
        batch, heads, tokens, dim = self.shape
        outputs = {
            p: self.recon[e].reshape(heads, batch, tokens, dim).permute(1, 0, 2, 3).to(self.dtype).contiguous()
            for e, p in enumerate(self.prefixes)
        }
        depth = self.prefixes[-1]
        indices = self.idx.reshape(heads, batch, tokens, depth).permute(1, 0, 2, 3).to(torch.uint8).contiguous()
        return outputs, indices


def _summary(sweep: _Sweep, initial, history, **head) -> dict[str, object]:
    final_objective, final_per_exit = sweep.objective()
    out = dict(head)
    out.update({
        "prefixes": list(sweep.prefixes),
        "exit_weights": list(sweep.weights),
        "initial_weighted_objective": initial[0],
        "final_weighted_objective": final_objective,
        "relative_objective_change": final_objective / max(initial[0], 1e-30) - 1.0,
        "initial_per_exit_mse": initial[1],
        "final_per_exit_mse": final_per_exit,
        "sweep_history": history,
    })
    return out


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
    """Reverse coordinate sweeps over the stages of ``initial_indices``
    ``[B,H,T,S]`` for ``states`` ``[B,H,T,D]``: each stage moves to the
    nearest codeword of its exact target, the others fixed.  Returns
    ``({prefix: reconstruction [B,H,T,D] in states' dtype}, uint8 indices
    [B,H,T,S], diagnostics)`` (nested_vq.py:583-741)."""

    if states.ndim != 4 or not torch.isfinite(states).all():
        raise ValueError("states must have finite [B,H,T,D] layout")
    prefixes, weights = _checked_exits(stage_tables, prefixes, exit_weights)
    if sweeps <= 0 or token_chunk_size <= 0:
        raise ValueError("coordinate sweeps and token chunks must be positive")
    sweep = _Sweep.build(states, stage_tables, initial_indices, prefixes, weights)
    initial = sweep.objective()
    history = []
    for number in range(1, sweeps + 1):
        changed: dict[str, float] = {}
        for stage in reversed(range(prefixes[-1])):
            slots = sweep.members(stage)
            if sweep.weight_sum(slots) <= 0:
                raise ValueError(f"stage {stage} is not covered by a positive exit")
            current = sweep.idx[..., stage].clone()
            chosen = _ops.nearest_f32(sweep.target(stage, slots, current), sweep.tables[stage])
            changed[str(stage + 1)] = float(chosen.ne(current).float().mean())
            sweep.move(slots, sweep.word(stage, chosen) - sweep.word(stage, current))
            sweep.idx[..., stage] = chosen
        weighted, per_exit = sweep.objective()
        history.append({
            "sweep": number,
            "weighted_objective": weighted,
            "per_exit_mse": per_exit,
            "changed_fraction_by_stage": changed,
            "mean_changed_fraction": sum(changed.values()) / len(changed),
        })
    outputs, indices = sweep.results()
    diagnostics = _summary(sweep, initial, history, mode="multi_exit_additive_coordinate",
                           coordinate_order="reverse", sweeps=sweeps)
    return outputs, indices, diagnostics


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
    """Reverse sweeps over the sliding stage pairs ``(S-1,S), ..., (1,2)``:
    each stage's shortlist is its current index and the ``shortlist_size - 1``
    nearest other codewords of its coordinate target, and the pair of
    shortlist entries with the lowest exact weighted error over the affected
    exits wins (the current pair on ties), so two indices can move together
    (nested_vq.py:757-1001).  Returns what the coordinate refinement returns,
    with the block diagnostics."""

    if states.ndim != 4 or not torch.isfinite(states).all():
        raise ValueError("states must have finite [B,H,T,D] layout")
    prefixes, weights = _checked_exits(stage_tables, prefixes, exit_weights)
    if sweeps <= 0 or shortlist_size < 2 or token_chunk_size <= 0:
        raise ValueError("invalid block-refinement search geometry")

    def depth_check(depth):
        if depth < 2:
            raise ValueError("two-stage refinement requires at least two stages")

    def table_check(stage, table):
        if table.shape[1] < shortlist_size or not torch.isfinite(table).all():
            raise ValueError(f"stage {stage} cannot support the requested shortlist")

    sweep = _Sweep.build(states, stage_tables, initial_indices, prefixes, weights, depth_check, table_check)
    if shortlist_size > 9:
        raise ValueError("the HIP shortlist search takes at most 8 alternatives (shortlist_size <= 9)")
    lib = _lib.load()
    heads, rows, dim = map(int, sweep.x.shape)
    stream = _lib.stream_handle(sweep.x.device)
    initial = sweep.objective()
    history = []
    for number in range(1, sweeps + 1):
        blocks = []
        for first in reversed(range(prefixes[-1] - 1)):
            pair = (first, first + 1)
            shortlists, current = [], []
            for stage in pair:
                slots = sweep.members(stage)
                if sweep.weight_sum(slots) <= 0:
                    raise ValueError(f"stage {stage} lacks a positive exit")
                cur = sweep.idx[..., stage].clone()
                others = _ops.nearest_topk_f32(sweep.target(stage, slots, cur), sweep.tables[stage],
                                               shortlist_size - 1, excluded=cur)
                shortlists.append(torch.cat((cur.unsqueeze(-1), others), dim=-1).contiguous())
                current.append(cur)
            slots = sweep.members(first)
            exit_slots, exit_weights, exit_second = _block_exits(slots, sweep, pair[1])
            chosen = [torch.empty_like(current[0]), torch.empty_like(current[1])]
            _lib.check(lib.jkv_pair_block_select(
                sweep.x.data_ptr(), sweep.recon.data_ptr(), int(sweep.recon.shape[0]), heads, rows, dim, len(slots),
                ctypes.addressof(exit_slots), ctypes.addressof(exit_weights), ctypes.addressof(exit_second),
                sweep.tables[pair[0]].data_ptr(), sweep.tables[pair[1]].data_ptr(),
                int(sweep.tables[pair[0]].shape[1]), int(sweep.tables[pair[1]].shape[1]),
                shortlists[0].data_ptr(), shortlists[1].data_ptr(), shortlist_size,
                chosen[0].data_ptr(), chosen[1].data_ptr(), stream))
            fractions = [float(c.ne(o).float().mean()) for c, o in zip(chosen, current)]
            for stage, c in zip(pair, chosen):
                sweep.idx[..., stage] = c
            blocks.append({"stages": [first + 1, first + 2], "changed_fraction": fractions})
        weighted, per_exit = sweep.objective()
        history.append({
            "sweep": number,
            "weighted_objective": weighted,
            "per_exit_mse": per_exit,
            "blocks": blocks,
            "mean_block_changed_fraction": sum(sum(b["changed_fraction"]) / 2 for b in blocks) / len(blocks),
        })
    outputs, indices = sweep.results()
    diagnostics = _summary(sweep, initial, history, mode="multi_exit_additive_block",
                           block_schedule="reverse_sliding_pairs", sweeps=sweeps, shortlist_size=shortlist_size)
    return outputs, indices, diagnostics


def _block_exits(slots: Sequence[int], sweep: _Sweep, second_stage: int):
    """Host arrays describing a block's weighted exits for
    ``jkv_pair_block_select``: stack slots, weights, and whether each exit
    also contains the second stage."""

    n = len(slots)
    return ((ctypes.c_int32 * n)(*slots),
            (ctypes.c_float * n)(*(sweep.weights[e] for e in slots)),
            (ctypes.c_int32 * n)(*(int(sweep.prefixes[e] > second_stage) for e in slots)))
