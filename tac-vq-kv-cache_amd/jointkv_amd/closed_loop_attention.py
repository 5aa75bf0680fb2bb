"""The closed-loop attention adapter: one decoder layer's self-attention with
its K/V routed through the codec, as the reference installs it for
calibration (experiments/train_full_model_closed_loop_vq.py:219-337,
``install_closed_loop_attention``; driven 32 layers deep by
experiments_followup_mistral/train_mistral_v_only.py:82-185).

Per layer: q/k/v projections of the hidden states, the codec on the raw
pre-RoPE K and V (``codec(layer, raw_key, raw_value, mode=...)`` ->
``QuantizedKV``), RoPE of q and K̂, ``repeat_kv``, SDPA with the model's
causal + sliding-window mask, and ``o_proj``.  Here the attention is the HIP
prefill kernel, and ``loss.backward()`` reaches the value tables through
its HIP value gradient (dV̂ = Pᵀ dO) and the codec's HIP scatter-add: the
V-only step's real upstream gradient, rather than a synthetic dL/dV̂.

The attention's backward is HIP too: the value leg alone when only the
tables need gradients, the full backward (query and key legs through the
rotary) when the hidden states require grad, so that stacked layers carry
the gradient down to lower layers' value tables as the reference's 32-layer
trajectory does.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .attention import MISTRAL_ROPE_THETA, MISTRAL_WINDOW, prefill_attention


@dataclass(frozen=True)
class AttentionWeights:
    """One layer's projections, ``[out, in]`` as ``nn.Linear`` stores them
    (Mistral-7B: q ``[4096,4096]``, k/v ``[1024,4096]``, o ``[4096,4096]``)."""

    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    o: torch.Tensor
    head_dim: int = 128

    @property
    def query_heads(self) -> int:
        return int(self.q.shape[0]) // self.head_dim

    @property
    def kv_heads(self) -> int:
        return int(self.k.shape[0]) // self.head_dim


def relative_trajectory_attention_mse(candidate: torch.Tensor, reference: torch.Tensor, *,
                                      epsilon: float = 1e-8) -> torch.Tensor:
    """mean((candidate - reference)^2) / max(mean(reference^2), epsilon), the
    reference output stopped (train_full_model_closed_loop_vq.py:200-216)."""

    if candidate.shape != reference.shape or candidate.ndim != 3:
        raise ValueError("trajectory attention outputs must share [B,T,D] geometry")
    if epsilon <= 0:
        raise ValueError("trajectory attention epsilon must be positive")
    target = reference.detach().float()
    return (candidate.float() - target).square().mean() / target.square().mean().clamp_min(epsilon)


def closed_loop_attention(
    hidden: torch.Tensor,
    weights: AttentionWeights,
    codec,
    layer: int,
    *,
    start_positions=0,
    mode: str = "uniform",
    window: int = MISTRAL_WINDOW,
    rope_theta: float = MISTRAL_ROPE_THETA,
    trajectory_epsilon: float | None = None,
    rate_records: list | None = None,
):
    """The quantized attention of ``layer`` over ``hidden`` ``[B,T,hidden]``
    fp16.  Returns the projected output ``[B,T,hidden]``, and with
    ``trajectory_epsilon`` also the layer's trajectory-match loss against the
    same attention on raw K/V (train_full_model_closed_loop_vq.py:304-334).
    A codec that returns projected depths has one rate record per request
    appended to ``rate_records`` (train_full_model_closed_loop_vq.py:261-273)."""

    batch, tokens, _ = map(int, hidden.shape)
    d = weights.head_dim
    query = F.linear(hidden, weights.q).view(batch, tokens, weights.query_heads, d).transpose(1, 2)
    raw_key = F.linear(hidden, weights.k).view(batch, tokens, weights.kv_heads, d).transpose(1, 2)
    raw_value = F.linear(hidden, weights.v).view(batch, tokens, weights.kv_heads, d).transpose(1, 2)
    quantized = codec(layer, raw_key, raw_value, mode=mode)
    if quantized.projected_depths is not None and rate_records is not None:
        depths = quantized.projected_depths
        for request, ledger in enumerate(depths.ledgers):
            rate_records.append({
                "layer": layer,
                "request": request,
                "total_bits": ledger.total_bits,
                "physical_effective_bits": ledger.physical_effective_bits,
                "low_blocks": depths.low_blocks_per_request[request],
                "anchor_blocks": depths.anchor_blocks_per_request[request],
                "high_blocks": depths.high_blocks_per_request[request],
            })
    out = prefill_attention(query, quantized.key, quantized.value, start_positions,
                            window=window, rope_theta=rope_theta)
    projected = F.linear(out.transpose(1, 2).contiguous().view(batch, tokens, -1), weights.o)
    if trajectory_epsilon is None:
        return projected
    with torch.no_grad():
        raw = prefill_attention(query, raw_key, raw_value, start_positions, window=window, rope_theta=rope_theta)
        raw_projected = F.linear(raw.transpose(1, 2).contiguous().view(batch, tokens, -1), weights.o)
    return projected, relative_trajectory_attention_mse(projected, raw_projected, epsilon=trajectory_epsilon)
