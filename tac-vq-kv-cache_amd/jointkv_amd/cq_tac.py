"""Grouped CQ hard encode/decode with straight-through gradients.

Drop-in for ``src/jointkv/cq_tac.py``: ``hard_grouped_cq`` (:33-114) and the
all-layer codec ``ClosedLoopGroupedCQ`` (:117-192).  One independent
nearest-codeword search per contiguous channel group; the search and the
decoded forward both use the fp16 round trip of the fp32 masters, and the
backward scatter-adds dL/dX̂ into the selected master centroids.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
import torch.nn as nn

from .closed_loop_vq import QuantizedKV, _run, hard_residual_vq_pair


def hard_grouped_cq(
    states: torch.Tensor,
    codebooks: torch.Tensor,
    *,
    selector_whiteners: torch.Tensor | None = None,
    token_chunk_size: int = 64,
    straight_through_states: bool = True,
    deterministic_backward: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Grouped composite quantization of states ``[B,H,T,D]`` against
    codebooks ``[H,G,K,S]`` (cq_tac.py:33-114): every S-wide channel group of
    a vector picks its nearest fp16-deployed codeword in one HIP launch.

    Returns (reconstruction ``[B,H,T,D]`` in ``states.dtype``, codes
    ``[B,H,T,G]`` uint8).  ``token_chunk_size`` is validated only; the kernel
    needs no row chunks.
    """

    if states.ndim != 4 or codebooks.ndim != 4:
        raise ValueError("states/codebooks must be [B,H,T,D]/[H,G,K,S]")
    batch, heads, tokens, dimension = map(int, states.shape)
    cb_heads, groups, clusters, subdimension = map(int, codebooks.shape)
    if cb_heads != heads or groups * subdimension != dimension:
        raise ValueError("CQ codebook geometry differs from states")
    if token_chunk_size <= 0:
        raise ValueError("token chunk size must be positive")
    if selector_whiteners is not None and tuple(selector_whiteners.shape) != (
        heads,
        groups,
        subdimension,
        subdimension,
    ):
        raise ValueError("CQ selector whitener geometry differs")
    tables = codebooks if codebooks.dtype == torch.float32 else codebooks.float()
    tables = tables.reshape(heads * groups, 1, clusters, subdimension).contiguous()
    whiteners = (
        None
        if selector_whiteners is None
        else selector_whiteners.detach().reshape(heads * groups, subdimension, subdimension)
    )
    outputs, codes = _run(
        states,
        tables,
        whiteners,
        groups,
        subdimension,
        (1,),
        straight_through_states,
        deterministic_backward,
    )
    return outputs[0], codes.reshape(batch, heads, tokens, groups)


def _is_identity(whitener: torch.Tensor) -> bool:
    size = whitener.shape[-1]
    eye = torch.eye(size, dtype=whitener.dtype, device=whitener.device)
    return bool(torch.equal(whitener, eye.expand_as(whitener)))


class ClosedLoopGroupedCQ(nn.Module):
    """Per-layer grouped-CQ codec: K codebooks are frozen buffers of the
    calibration, V codebooks are the trainable fp32 masters.

    Same constructor, buffers, parameters and forward contract as
    cq_tac.py:117-192.  An identity selector whitener (the default the
    reference substitutes when a parent has none, train_mistral_v_only.py:69)
    selects exactly the same codes as no whitener, so it is recognised once
    at construction and the unwhitened kernel runs.
    """

    def __init__(
        self,
        key_codebooks: Sequence[torch.Tensor],
        value_codebooks: Sequence[torch.Tensor],
        key_selector_whiteners: Sequence[torch.Tensor],
        *,
        dynamic_bpa: float,
        token_chunk_size: int = 64,
    ) -> None:
        super().__init__()
        if not (
            len(key_codebooks) == len(value_codebooks) == len(key_selector_whiteners)
        ) or not key_codebooks:
            raise ValueError("CQ layer payloads differ")
        geometry = tuple(key_codebooks[0].shape)
        if len(geometry) != 4 or any(
            tuple(row.shape) != geometry for row in (*key_codebooks, *value_codebooks)
        ):
            raise ValueError("CQ codebook layers have inconsistent geometry")
        if any(
            tuple(row.shape) != (geometry[0], geometry[1], geometry[3], geometry[3])
            for row in key_selector_whiteners
        ):
            raise ValueError("CQ key selector layers have inconsistent geometry")
        self.key_tables = nn.ParameterList(
            [nn.Parameter(row.detach().float().contiguous(), requires_grad=False) for row in key_codebooks]
        )
        self.value_tables = nn.ParameterList(
            [nn.Parameter(row.detach().float().contiguous()) for row in value_codebooks]
        )
        self._identity_selector: list[bool] = []
        for layer, whitener in enumerate(key_selector_whiteners):
            value = whitener.detach().float().contiguous()
            self.register_buffer(f"key_selector_whitener_{layer:02d}", value, persistent=True)
            self._identity_selector.append(_is_identity(value))
        self.dynamic_bpa = float(dynamic_bpa)
        self.token_chunk_size = int(token_chunk_size)

    def key_whitener(self, layer: int) -> torch.Tensor:
        return getattr(self, f"key_selector_whitener_{layer:02d}")

    def forward(
        self,
        layer: int,
        raw_key: torch.Tensor,
        raw_value: torch.Tensor,
        *,
        mode: str = "uniform",
    ) -> QuantizedKV:
        if mode != "uniform":
            raise ValueError("grouped CQ supports one fixed-rate uniform mode")
        whitener = None if self._identity_selector[layer] else self.key_whitener(layer)
        kt, vt = self.key_tables[layer], self.value_tables[layer]
        heads, groups, _k, sub = map(int, kt.shape)
        if (whitener is None and raw_key.shape == raw_value.shape and raw_key.dtype == raw_value.dtype
                and raw_key.ndim == 4 and raw_key.shape[1] == heads and raw_key.shape[3] == groups * sub):
            # one launch for the layer's K and V (same bits as two encodes)
            kx, kc, vx, vc = hard_residual_vq_pair(raw_key, raw_value, kt.unsqueeze(2), vt.unsqueeze(2),
                                                   prefixes=(1,))
            key, key_indices, value, value_indices = kx[1], kc[..., 0], vx[1], vc[..., 0]
        else:
            key, key_indices = hard_grouped_cq(
                raw_key,
                kt,
                selector_whiteners=whitener,
                token_chunk_size=self.token_chunk_size,
            )
            value, value_indices = hard_grouped_cq(
                raw_value,
                vt,
                token_chunk_size=self.token_chunk_size,
            )
        return QuantizedKV(
            key=key,
            value=value,
            key_indices=key_indices,
            value_indices=value_indices,
            projected_depths=None,
        )
