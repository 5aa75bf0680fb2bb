"""Hard residual VQ with straight-through gradients on gfx950 kernels.

Drop-in for the hot subset of ``src/jointkv/closed_loop_vq.py``:
``QuantizedKV`` (:43-49) and ``hard_residual_vq_exits`` (:235-410), plus the
grouped residual geometry (per-(head, group) residual stages) that the same
function expresses when heads and channel groups are folded together, and the
frozen-code decode of
``experiments/train_pure_uniform16_closed_loop_vq.py:395-442``.

Forward: one HIP launch searches every stage (fp16-deployed codewords,
fp32 residuals, lowest index on ties) and writes uint8 codes plus the fp16
reconstruction at each requested prefix.  Backward: one HIP launch
scatter-adds dL/dX̂ into the fp32 masters of every selected codeword (the
backward of the reference's ``torch.gather`` through its deploy STE at :298),
and the identity straight-through edge hands dL/dX̂ to the states (:408).
"""

from __future__ import annotations

from dataclasses import dataclass
import math
from typing import Sequence

import torch

from . import _ops


@dataclass(frozen=True)
class QuantizedKV:
    """Result type of the codec modules (closed_loop_vq.py:43-49)."""

    key: torch.Tensor
    value: torch.Tensor
    key_indices: torch.Tensor
    value_indices: torch.Tensor
    projected_depths: object | None


class _HardResidualVQ(torch.autograd.Function):
    """Autograd node: HIP encode forward, HIP scatter-add backward."""

    @staticmethod
    def forward(ctx, states, tables, whiteners, groups, group_dim, exits, straight_through, deterministic):
        recon, codes = _ops.rvq_encode(
            states.detach(),
            tables.detach(),
            groups=groups,
            group_dim=group_dim,
            exits=exits,
            whiteners=whiteners,
        )
        ctx.save_for_backward(codes)
        ctx.exits = tuple(exits)
        ctx.group_dim = group_dim
        ctx.table_shape = tables.shape
        ctx.straight_through = straight_through
        ctx.deterministic = deterministic
        ctx.mark_non_differentiable(codes)
        return (*recon, codes)

    @staticmethod
    def backward(ctx, *grad_outputs):
        (codes,) = ctx.saved_tensors
        grad_states, grad_tables = _table_and_state_grads(
            ctx, grad_outputs[:-1], codes, ctx.table_shape, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return grad_states, grad_tables, None, None, None, None, None, None


def _table_and_state_grads(ctx, grads, codes, table_shape, need_states, need_tables):
    """The straight-through backward of one encode: the summed upstream
    gradient for the states and the scatter-add into the table masters."""

    live = [(g, e) for g, e in zip(grads, ctx.exits) if g is not None]
    grad_states = grad_tables = None
    if live and need_states and ctx.straight_through:
        # the summed exit gradients (one exit: its gradient itself; the sums
        # are out of place, so no caller's tensor is modified)
        grad_states = live[0][0]
        for g, _ in live[1:]:
            grad_states = grad_states + g
    if live and need_tables:
        grad_tables = torch.zeros(table_shape, dtype=torch.float32, device=codes.device)
        _ops.rvq_scatter_grad(
            [g for g, _ in live],
            [e for _, e in live],
            codes,
            grad_tables,
            group_dim=ctx.group_dim,
            deterministic=ctx.deterministic,
        )
    return grad_states, grad_tables


class _HardResidualVQPair(torch.autograd.Function):
    """A layer's K and V through one HIP launch (same geometry, no
    whitener); the backward is each side's own straight-through scatter."""

    @staticmethod
    def forward(ctx, key_states, value_states, key_tables, value_tables, groups, group_dim, exits,
                straight_through, deterministic):
        rk, ck, rv, cv = _ops.rvq_encode_kv(
            key_states.detach(),
            value_states.detach(),
            key_tables.detach(),
            value_tables.detach(),
            groups=groups,
            group_dim=group_dim,
            exits=exits,
        )
        ctx.save_for_backward(ck, cv)
        ctx.exits = tuple(exits)
        ctx.group_dim = group_dim
        ctx.table_shapes = (key_tables.shape, value_tables.shape)
        ctx.straight_through = straight_through
        ctx.deterministic = deterministic
        ctx.mark_non_differentiable(ck, cv)
        # a side whose states and tables take no gradient gives outputs that
        # take none either (as its own encode would), so that nothing
        # downstream forms a gradient for them
        need = ctx.needs_input_grad
        if not (need[0] or need[2]):
            ctx.mark_non_differentiable(*rk)
        if not (need[1] or need[3]):
            ctx.mark_non_differentiable(*rv)
        return (*rk, *rv, ck, cv)

    @staticmethod
    def backward(ctx, *grad_outputs):
        ck, cv = ctx.saved_tensors
        n = len(ctx.exits)
        need = ctx.needs_input_grad
        gsk, gtk = _table_and_state_grads(ctx, grad_outputs[:n], ck, ctx.table_shapes[0], need[0], need[2])
        gsv, gtv = _table_and_state_grads(ctx, grad_outputs[n:2 * n], cv, ctx.table_shapes[1], need[1], need[3])
        return gsk, gsv, gtk, gtv, None, None, None, None, None


def hard_residual_vq_pair(
    key_states: torch.Tensor,
    value_states: torch.Tensor,
    key_tables: torch.Tensor,
    value_tables: torch.Tensor,
    *,
    prefixes: Sequence[int],
    straight_through_states: bool = True,
    deterministic_backward: bool = False,
):
    """A layer's K and V encode in one launch, for the codec forward
    (uniform_depth_tac.py:69-101 encodes K, then V, with one geometry).

    ``*_states[B,H,T,G*d]`` share shape and dtype; ``*_tables`` are
    ``[H,G,S,K,d]`` (grouped) or ``[H,S,K,D]`` (one group), fp32 masters, no
    whitener.  Returns ``(key exits, key codes, value exits, value codes)``
    as :func:`hard_grouped_residual_vq` (grouped) or
    :func:`hard_residual_vq_exits` would, with the same bits.
    """

    if key_states.shape != value_states.shape or key_states.dtype != value_states.dtype:
        raise ValueError("K and V states must share their geometry")
    if key_tables.shape != value_tables.shape or key_states.ndim != 4 or key_tables.ndim not in (4, 5):
        raise ValueError("K and V tables must share their geometry")
    batch, heads, tokens, dimension = map(int, key_states.shape)
    if key_tables.ndim == 5:
        t_heads, groups, stages, clusters, group_dim = map(int, key_tables.shape)
    else:
        t_heads, stages, clusters, group_dim = map(int, key_tables.shape)
        groups = 1
    if t_heads != heads or groups * group_dim != dimension:
        raise ValueError("state and table geometry differs")
    requested = tuple(sorted(set(int(depth) for depth in prefixes)))
    if not requested or requested[0] <= 0 or requested[-1] > stages:
        raise ValueError("requested prefixes lie outside the VQ ladder")

    def flat(tables):
        t = tables if tables.dtype == torch.float32 else tables.float()
        return t.reshape(heads * groups, stages, clusters, group_dim).contiguous()

    outputs = _HardResidualVQPair.apply(
        key_states, value_states, flat(key_tables), flat(value_tables), groups, group_dim, requested,
        straight_through_states, deterministic_backward,
    )
    n = len(requested)
    kc, vc = outputs[2 * n], outputs[2 * n + 1]
    if groups == 1 and key_tables.ndim == 4:
        kc = kc.reshape(batch, heads, tokens, stages)
        vc = vc.reshape(batch, heads, tokens, stages)
    return dict(zip(requested, outputs[:n])), kc, dict(zip(requested, outputs[n:2 * n])), vc


def _validate_soft_backward(topk: int, temperature: float, beta: float, cardinality: int) -> None:
    # closed_loop_vq.py:273-284
    if topk <= 0 or topk > cardinality:
        raise ValueError("soft-backward top-k lies outside the codebook")
    if not math.isfinite(beta) or beta < 0:
        raise ValueError("soft-backward beta must be finite and non-negative")
    if beta > 0 and topk <= 1:
        raise ValueError("positive soft-backward beta requires top-k > 1")
    if beta > 0 and (not math.isfinite(temperature) or temperature <= 0):
        raise ValueError("soft-backward temperature must be finite and positive")
    if beta > 0:
        raise NotImplementedError(
            "the top-k soft-assignment surrogate backward is outside the gfx950 hot path"
        )


def _run(states, tables_f32, whiteners, groups, group_dim, exits, straight_through, deterministic):
    outputs = _HardResidualVQ.apply(
        states, tables_f32, whiteners, groups, group_dim, tuple(exits), straight_through, deterministic
    )
    return list(outputs[:-1]), outputs[-1]


def hard_residual_vq_exits(
    states: torch.Tensor,
    tables: torch.Tensor,
    *,
    prefixes: Sequence[int],
    assignment_whiteners: torch.Tensor | None = None,
    token_chunk_size: int = 1024,
    straight_through_states: bool = True,
    soft_backward_topk: int = 1,
    soft_backward_temperature: float = 0.0,
    soft_backward_beta: float = 0.0,
    deterministic_backward: bool = False,
) -> tuple[dict[int, torch.Tensor], torch.Tensor]:
    """Greedy residual VQ of every head vector through all S stages in one
    HIP launch, with straight-through exits at the requested depths.

    Same contract as closed_loop_vq.py:235-410: ``states[B,H,T,D]``,
    ``tables[H,S,K,D]`` (fp32 masters; search and decode use their fp16
    round trip), returns ``({depth: [B,H,T,D] in states.dtype}, uint8
    [B,H,T,S])``.  ``token_chunk_size`` is validated and otherwise unused:
    the kernel has no host-side chunk loop.
    """

    if states.ndim != 4 or tables.ndim != 4:
        raise ValueError("states/tables must have [B,H,T,D]/[H,S,K,D]")
    batch, heads, tokens, dimension = map(int, states.shape)
    if tables.shape[0] != heads or tables.shape[-1] != dimension:
        raise ValueError("state and table geometry differs")
    requested = tuple(sorted(set(int(depth) for depth in prefixes)))
    stages = int(tables.shape[1])
    if not requested or requested[0] <= 0 or requested[-1] > stages:
        raise ValueError("requested prefixes lie outside the VQ ladder")
    if assignment_whiteners is not None and tuple(assignment_whiteners.shape) != (
        heads,
        dimension,
        dimension,
    ):
        raise ValueError("assignment whitener has invalid geometry")
    _validate_soft_backward(
        soft_backward_topk, soft_backward_temperature, soft_backward_beta, int(tables.shape[2])
    )
    if token_chunk_size <= 0:
        raise ValueError("token chunk size must be positive")
    tables_f32 = tables if tables.dtype == torch.float32 else tables.float()
    tables_f32 = tables_f32.contiguous()
    outputs, codes = _run(
        states,
        tables_f32,
        None if assignment_whiteners is None else assignment_whiteners.detach(),
        1,
        dimension,
        requested,
        straight_through_states,
        deterministic_backward,
    )
    return dict(zip(requested, outputs)), codes.reshape(batch, heads, tokens, stages)


def hard_grouped_residual_vq(
    states: torch.Tensor,
    tables: torch.Tensor,
    *,
    prefixes: Sequence[int],
    assignment_whiteners: torch.Tensor | None = None,
    straight_through_states: bool = True,
    deterministic_backward: bool = False,
) -> tuple[dict[int, torch.Tensor], torch.Tensor]:
    """Grouped residual VQ: ``states[B,H,T,G*d]``, ``tables[H,G,S,K,d]``.

    Each (head, group) channel slice runs its own S-stage greedy residual
    search.  This is exactly ``hard_residual_vq_exits`` applied to the
    folded view ``states.view(B,H,T,G,d).permute(0,1,3,2,4).reshape(B,H*G,T,d)``
    with ``tables.reshape(H*G,S,K,d)``, with the codes unfolded to
    ``[B,H,T,G,S]`` and the reconstruction refolded to ``[B,H,T,G*d]``; the
    kernel reads the strided slices directly instead of materialising the
    permuted copy.  ``assignment_whiteners`` is ``[H,G,d,d]`` or None.
    """

    if states.ndim != 4 or tables.ndim != 5:
        raise ValueError("states/tables must have [B,H,T,G*d]/[H,G,S,K,d]")
    batch, heads, tokens, dimension = map(int, states.shape)
    t_heads, groups, stages, clusters, group_dim = map(int, tables.shape)
    if t_heads != heads or groups * group_dim != dimension:
        raise ValueError("state and table geometry differs")
    requested = tuple(sorted(set(int(depth) for depth in prefixes)))
    if not requested or requested[0] <= 0 or requested[-1] > stages:
        raise ValueError("requested prefixes lie outside the VQ ladder")
    whiteners = None
    if assignment_whiteners is not None:
        if tuple(assignment_whiteners.shape) != (heads, groups, group_dim, group_dim):
            raise ValueError("assignment whitener has invalid geometry")
        whiteners = assignment_whiteners.detach().reshape(heads * groups, group_dim, group_dim)
    tables_f32 = tables if tables.dtype == torch.float32 else tables.float()
    tables_f32 = tables_f32.reshape(heads * groups, stages, clusters, group_dim).contiguous()
    outputs, codes = _run(
        states,
        tables_f32,
        whiteners,
        groups,
        group_dim,
        requested,
        straight_through_states,
        deterministic_backward,
    )
    return dict(zip(requested, outputs)), codes


def frozen_assignment_reconstruction(
    states: torch.Tensor,
    tables: torch.Tensor,
    indices: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Decode literal codes with the identity STE (no nearest-neighbour search).

    Mirrors ``frozen_assignment_u16_reconstruction``
    (experiments/train_pure_uniform16_closed_loop_vq.py:395-442) for any
    depth: ``states[B,H,T,D]``, ``tables[H,S,K,D]``, ``indices[B,H,T,S]``.
    Returns the reconstruction (+ identity edge to ``states``) and the
    indices as uint8.  Gradients reach the selected fp32 master words.
    """

    if states.ndim != 4 or tables.ndim != 4 or indices.ndim != 4:
        raise ValueError("frozen assignment geometry must be [B,H,T,D]/[H,S,K,D]/[B,H,T,S]")
    batch, heads, tokens, dimension = map(int, states.shape)
    stages = int(tables.shape[1])
    if int(tables.shape[0]) != heads or int(tables.shape[-1]) != dimension:
        raise ValueError("frozen assignment table geometry differs")
    if tuple(indices.shape) != (batch, heads, tokens, stages):
        raise ValueError("frozen assignment indices differ from live raw geometry")
    cardinality = int(tables.shape[2])
    device_indices = indices.to(device=states.device)
    if int(device_indices.min()) < 0 or int(device_indices.max()) >= cardinality:
        raise ValueError("frozen assignment index lies outside codebook")
    codes = device_indices.to(torch.uint8).reshape(batch, heads, tokens, 1, stages).contiguous()
    tables_f32 = (tables if tables.dtype == torch.float32 else tables.float()).contiguous()
    out = _FrozenDecode.apply(states, tables_f32, codes, stages)
    return out, codes.reshape(batch, heads, tokens, stages)


class _FrozenDecode(torch.autograd.Function):
    @staticmethod
    def forward(ctx, states, tables, codes, depth):
        out = _ops.rvq_decode(codes, tables.detach(), depth=depth, dtype=states.dtype)
        ctx.save_for_backward(codes)
        ctx.table_shape = tables.shape
        ctx.depth = depth
        ctx.group_dim = int(tables.shape[-1])
        return out

    @staticmethod
    def backward(ctx, grad):
        (codes,) = ctx.saved_tensors
        grad_tables = None
        if ctx.needs_input_grad[1]:
            grad_tables = torch.zeros(ctx.table_shape, dtype=torch.float32, device=grad.device)
            _ops.rvq_scatter_grad([grad], [ctx.depth], codes, grad_tables, group_dim=ctx.group_dim)
        grad_states = grad if ctx.needs_input_grad[0] else None
        return grad_states, grad_tables, None, None
