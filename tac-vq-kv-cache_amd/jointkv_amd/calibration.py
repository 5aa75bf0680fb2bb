"""Codebook-gradient clipping and plain SGD for the V-codebook calibration step.

``clip_codebook_gradients`` keeps the contract of
``experiments/train_pure_uniform16_closed_loop_vq.py:1151-1304`` (modes
``global``, ``per_layer_kv``, ``key_global_value_per_layer``; same audit
dictionary; same error texts), but computes every table norm in one fp64
device reduction and applies every scale in one launch, so the whole clip
costs two small device-to-host copies instead of one sync per table.  The
scale follows ``torch.nn.utils.clip_grad_norm_``:
``min(1, max_norm / (total_norm + 1e-6))`` in fp32, multiplied into the
gradient even when it equals one.
"""

from __future__ import annotations

import math
from typing import Any, Sequence

import numpy as np
import torch

from . import _ops

_F32 = np.float32


def _norms(tensors: Sequence[torch.Tensor | None]) -> list[float]:
    """fp32 L2 norms (as Python floats) of the given gradients; None -> 0."""

    live = [t for t in tensors if t is not None]
    if not live:
        return [0.0 for _ in tensors]
    sums = _ops.sumsq(live).cpu().numpy()
    values = iter(np.sqrt(sums).astype(_F32).tolist())
    return [0.0 if t is None else float(next(values)) for t in tensors]


def _clip_coef(norms: Sequence[float], maximum_norm: float) -> tuple[float, float]:
    """torch clip_grad_norm_: total = ||(n_1..n_k)||, coef = min(1, max/(total+1e-6))."""

    total = _F32(math.sqrt(sum(float(_F32(n)) ** 2 for n in norms)))
    coef = _F32(maximum_norm) / (total + _F32(1e-6))
    return float(total), float(min(coef, _F32(1.0)))


def _scale(grads: Sequence[torch.Tensor], scales: Sequence[float]) -> None:
    if grads:
        _ops.scale_sgd(list(grads), list(scales))


def clip_codebook_gradients(codec, *, maximum_norm: float, mode: str) -> dict[str, Any]:
    """Clip codebook gradients without ever amplifying a small group."""

    if not math.isfinite(maximum_norm) or maximum_norm <= 0:
        raise ValueError("gradient cap must be finite and positive")
    groups = [
        (layer, kind, parameter)
        for kind, tables in (("key", codec.key_tables), ("value", codec.value_tables))
        for layer, parameter in enumerate(tables)
    ]
    if mode == "global":
        parameters = [p for _l, _k, p in groups if p.requires_grad]
        if not parameters:
            raise RuntimeError("gradient clipping received no trainable codebooks")
        grads = [p.grad for p in parameters if p.grad is not None]
        norms = _norms(grads)
        total_before, coef = _clip_coef(norms, maximum_norm) if grads else (0.0, 1.0)
        _scale(grads, [coef] * len(grads))
        scale = min(1.0, maximum_norm / (total_before + 1e-12))
        return {
            "mode": mode,
            "maximum_norm": float(maximum_norm),
            "group_count": len(groups),
            "trainable_group_count": len(parameters),
            "total_norm_before_clip": total_before,
            "total_norm_after_clip": min(total_before, maximum_norm),
            "global_scale": scale,
            "per_group": None,
        }
    if mode not in {"per_layer_kv", "key_global_value_per_layer"}:
        raise ValueError(f"unknown gradient clip mode: {mode}")

    all_grads = [p.grad for _l, _k, p in groups]
    before = _norms(all_grads)
    scales = [1.0] * len(groups)
    key_rows = [i for i, row in enumerate(groups) if row[1] == "key"]
    value_rows = [i for i, row in enumerate(groups) if row[1] == "value"]
    key_total_before = 0.0
    key_parameters = []
    if mode == "key_global_value_per_layer":
        key_parameters = [groups[i][2] for i in key_rows if groups[i][2].requires_grad]
        key_total_before = math.sqrt(sum(before[i] * before[i] for i in key_rows))
        live = [i for i in key_rows if groups[i][2].requires_grad and groups[i][2].grad is not None]
        if live:
            _total, coef = _clip_coef([before[i] for i in live], maximum_norm)
            for i in live:
                scales[i] = coef
        per_table = value_rows
    else:
        per_table = list(range(len(groups)))
    for i in per_table:
        if groups[i][2].grad is not None:
            _total, scales[i] = _clip_coef([before[i]], maximum_norm)
    touched = [i for i in range(len(groups)) if groups[i][2].grad is not None and (
        i in per_table or (mode == "key_global_value_per_layer" and groups[i][2].requires_grad))]
    _scale([groups[i][2].grad for i in touched], [scales[i] for i in touched])
    after = _norms(all_grads)

    rows: list[dict[str, Any]] = []
    squared_before = squared_after = 0.0
    for i, (layer, kind, parameter) in enumerate(groups):
        b, a = before[i], after[i]
        squared_before += b * b
        squared_after += a * a
        row = {
            "layer": layer,
            "kind": kind,
            "norm_before_clip": b,
            "norm_after_clip": a,
            "scale": 1.0 if b == 0.0 else a / b,
        }
        if mode == "key_global_value_per_layer" and kind == "key":
            row["clip_activated"] = key_total_before > maximum_norm
            row["shared_group"] = "all_key_tables"
        else:
            row["clip_activated"] = b > maximum_norm
            if mode == "key_global_value_per_layer":
                row["shared_group"] = None
        rows.append(row)
    result: dict[str, Any] = {
        "mode": mode,
        "maximum_norm": float(maximum_norm),
        "group_count": (1 + len(value_rows)) if mode == "key_global_value_per_layer" else len(groups),
        "trainable_group_count": (
            int(bool(key_parameters)) + sum(groups[i][2].requires_grad for i in value_rows)
            if mode == "key_global_value_per_layer"
            else sum(p.requires_grad for _l, _k, p in groups)
        ),
        "total_norm_before_clip": math.sqrt(squared_before),
        "total_norm_after_clip": math.sqrt(squared_after),
        "global_scale": None,
        "per_group": rows,
    }
    if mode == "key_global_value_per_layer":
        result["key_global_norm_before_clip"] = key_total_before
    return result


def sgd_step(parameters: Sequence[torch.Tensor], *, lr: float) -> None:
    """Plain SGD ``p -= lr * p.grad`` (no momentum, no weight decay) in one launch.

    Same update as ``torch.optim.SGD(params, lr)`` used by
    ``experiments_followup_mistral/train_mistral_v_only.py:128,153``.
    """

    live = [p for p in parameters if p.grad is not None]
    if not live:
        return
    with torch.no_grad():
        _ops.scale_sgd([p.grad for p in live], [1.0] * len(live), params=[p.data for p in live], lr=lr)
