"""Uniform-depth residual-VQ codec with frozen K and trainable V tables.

Drop-in for ``src/jointkv/uniform_depth_tac.py`` (``ClosedLoopUniformResidualVQ``
:19-101): same constructor checks and error texts, same parameter and buffer
names, same ``forward(layer, raw_key, raw_value, mode=...)`` -> QuantizedKV.
Optionally the tables may carry a channel-group axis (``[H,G,S,K,d]``), in
which case every (head, group) slice is its own residual problem.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
import torch.nn as nn

from .closed_loop_vq import QuantizedKV, hard_grouped_residual_vq, hard_residual_vq_exits, hard_residual_vq_pair


class ClosedLoopUniformResidualVQ(nn.Module):
    """Per-layer residual-VQ codec at one fixed depth: every stage of every
    K and V head vector is coded (hard), and only the V tables train."""

    def __init__(
        self,
        key_tables: Sequence[torch.Tensor],
        value_tables: Sequence[torch.Tensor],
        key_whiteners: Sequence[torch.Tensor | None],
        *,
        depth: int,
        dynamic_bpa: float,
        token_chunk_size: int = 1024,
    ) -> None:
        super().__init__()
        if depth <= 0 or dynamic_bpa <= 0 or token_chunk_size <= 0:
            raise ValueError("invalid uniform residual-VQ configuration")
        if not key_tables or not (len(key_tables) == len(value_tables) == len(key_whiteners)):
            raise ValueError("uniform residual-VQ layer payloads differ")
        geometry = tuple(key_tables[0].shape)
        grouped = len(geometry) == 5
        stage_axis = 2 if grouped else 1
        if len(geometry) not in (4, 5) or geometry[stage_axis] != depth:
            raise ValueError("uniform residual-VQ tables have the wrong depth")
        if geometry[stage_axis + 1] != 256:
            raise ValueError("this deployment contract requires 8-bit stage indices")
        if any(tuple(table.shape) != geometry for table in (*key_tables, *value_tables)):
            raise ValueError("uniform residual-VQ layer geometries differ")
        self.key_tables = nn.ParameterList(
            [nn.Parameter(table.detach().float().contiguous(), requires_grad=False) for table in key_tables]
        )
        self.value_tables = nn.ParameterList(
            [nn.Parameter(table.detach().float().contiguous()) for table in value_tables]
        )
        heads, dimension = geometry[0], geometry[-1]
        whitener_shape = (heads, geometry[1], dimension, dimension) if grouped else (heads, dimension, dimension)
        for layer, whitener in enumerate(key_whiteners):
            if whitener is not None and tuple(whitener.shape) != whitener_shape:
                raise ValueError("key assignment whitener geometry differs")
            self.register_buffer(
                f"key_whitener_{layer:02d}",
                torch.empty(0, dtype=torch.float32)
                if whitener is None
                else whitener.detach().float().contiguous(),
                persistent=True,
            )
        self.grouped = grouped
        self.depth = int(depth)
        self.dynamic_bpa = float(dynamic_bpa)
        self.token_chunk_size = int(token_chunk_size)

    def whitener(self, layer: int) -> torch.Tensor | None:
        value = getattr(self, f"key_whitener_{layer:02d}")
        return None if value.numel() == 0 else value

    def _encode(self, states, tables, whitener):
        if self.grouped:
            exits, indices = hard_grouped_residual_vq(
                states, tables, prefixes=(self.depth,), assignment_whiteners=whitener
            )
        else:
            exits, indices = hard_residual_vq_exits(
                states,
                tables,
                prefixes=(self.depth,),
                assignment_whiteners=whitener,
                token_chunk_size=self.token_chunk_size,
            )
        return exits[self.depth], indices

    def forward(
        self,
        layer: int,
        raw_key: torch.Tensor,
        raw_value: torch.Tensor,
        *,
        mode: str = "uniform",
    ) -> QuantizedKV:
        if mode != "uniform":
            raise ValueError("uniform residual VQ exposes only uniform mode")
        whitener = self.whitener(layer)
        if whitener is None and raw_key.shape == raw_value.shape and raw_key.dtype == raw_value.dtype:
            # one launch for the layer's K and V (same bits as two encodes)
            kx, key_indices, vx, value_indices = hard_residual_vq_pair(
                raw_key, raw_value, self.key_tables[layer], self.value_tables[layer], prefixes=(self.depth,))
            key, value = kx[self.depth], vx[self.depth]
        else:
            key, key_indices = self._encode(raw_key, self.key_tables[layer], whitener)
            value, value_indices = self._encode(raw_value, self.value_tables[layer], None)
        return QuantizedKV(
            key=key,
            value=value,
            key_indices=key_indices,
            value_indices=value_indices,
            projected_depths=None,
        )
