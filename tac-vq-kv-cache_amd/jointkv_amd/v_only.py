"""The V-only calibration step over a stack of decoder layers.

Drop-in for the training loop of
``experiments_followup_mistral/train_mistral_v_only.py:119-163`` with the
attention adapter of ``experiments/train_full_model_closed_loop_vq.py``
(``ClosedLoopRunContext`` :178-197, ``causal_loss`` :359-364, ``run_loss``
:367-377).  The backbone is frozen; only the codec's fp32 value masters
train.  One step, in the reference's order:

  zero the value gradients -> forward with every layer's K/V routed through
  the codec -> causal loss -> "nonfinite loss or unexpected rate" check ->
  backward -> "nonfinite/missing V gradient" check -> per_layer_kv clip at
  1.0 -> SGD at lr 0.001.

On gfx950 every codec and attention op of the step is a HIP launch: the
grouped residual encode of K and V, the prefill attention with its log-sum-
exp, its backward (value leg; query and key legs above the first layer,
where the hidden states carry gradient), the scatter-add of dL/dV̂ into the
value masters, and the fused norm/clip/SGD launches.  The frozen backbone's
own dense layers (projections, RMSNorm, MLP, embedding, lm_head) are
ordinary PyTorch ops on the same stream.

``DecoderStack`` is the Mistral decoder restated over plain weight tensors
(pre-norm blocks: attention then gated-SiLU MLP, each added to the residual),
so that a synthetic stack of any depth can stand in for the 32-layer model
the reference loads from disk.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Sequence

import torch
import torch.nn.functional as F

from .attention import MISTRAL_ROPE_THETA, MISTRAL_WINDOW
from .calibration import clip_codebook_gradients, sgd_step
from .closed_loop_attention import AttentionWeights, closed_loop_attention

MISTRAL_RMS_EPS = 1e-5


class ClosedLoopRunContext:
    """The codec, its mode and the rate records of one forward
    (train_full_model_closed_loop_vq.py:178-197)."""

    def __init__(self, codec, mode: str) -> None:
        self.codec = codec
        self.mode = mode
        self.rate_records: list[dict[str, Any]] = []

    def reset(self, mode: str) -> None:
        self.mode = mode
        self.rate_records.clear()


@dataclass(frozen=True)
class DecoderLayerWeights:
    """One Mistral decoder layer: RMSNorm weights ``[hidden]``, the attention
    projections and the MLP ``gate``/``up`` ``[inter,hidden]`` and ``down``
    ``[hidden,inter]`` (``nn.Linear`` layout)."""

    input_norm: torch.Tensor
    attention: AttentionWeights
    post_attention_norm: torch.Tensor
    gate: torch.Tensor
    up: torch.Tensor
    down: torch.Tensor


@dataclass(frozen=True)
class DecoderStack:
    """Embedding ``[vocab,hidden]``, decoder layers, final RMSNorm and
    ``lm_head`` ``[vocab,hidden]``, all fp16 and frozen."""

    embed: torch.Tensor
    layers: tuple[DecoderLayerWeights, ...]
    final_norm: torch.Tensor
    lm_head: torch.Tensor
    rms_eps: float = MISTRAL_RMS_EPS
    window: int = MISTRAL_WINDOW
    rope_theta: float = MISTRAL_ROPE_THETA

    @classmethod
    def synthetic(cls, generator: torch.Generator, *, layers: int, hidden: int, kv_heads: int,
                  intermediate: int, vocab: int, head_dim: int = 128, window: int = MISTRAL_WINDOW,
                  rope_theta: float = MISTRAL_ROPE_THETA) -> "DecoderStack":
        """Random fp16 weights of the given shape (N(0, 1/fan_in) matrices,
        norm weights near 1), drawn on the generator's device; move with
        :meth:`to`."""

        if hidden % head_dim or layers <= 0 or kv_heads <= 0 or (hidden // head_dim) % kv_heads:
            raise ValueError("invalid synthetic decoder geometry")

        dev = generator.device

        def mat(rows, cols):
            return (torch.randn(rows, cols, generator=generator, device=dev) / cols ** 0.5).half()

        def norm():
            return (1.0 + 0.1 * torch.randn(hidden, generator=generator, device=dev)).half()

        stack = []
        for _ in range(layers):
            attention = AttentionWeights(mat(hidden, hidden), mat(head_dim * kv_heads, hidden),
                                         mat(head_dim * kv_heads, hidden), mat(hidden, hidden), head_dim)
            stack.append(DecoderLayerWeights(norm(), attention, norm(), mat(intermediate, hidden),
                                             mat(intermediate, hidden), mat(hidden, intermediate)))
        return cls(torch.randn(vocab, hidden, generator=generator, device=dev).half(), tuple(stack), norm(),
                   mat(vocab, hidden), window=window, rope_theta=rope_theta)

    def to(self, device) -> "DecoderStack":
        def move(t):
            return t.to(device)

        layers = tuple(
            DecoderLayerWeights(move(w.input_norm),
                                AttentionWeights(move(w.attention.q), move(w.attention.k), move(w.attention.v),
                                                 move(w.attention.o), w.attention.head_dim),
                                move(w.post_attention_norm), move(w.gate), move(w.up), move(w.down))
            for w in self.layers)
        return DecoderStack(move(self.embed), layers, move(self.final_norm), move(self.lm_head),
                            self.rms_eps, self.window, self.rope_theta)


def rms_norm(hidden: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Mistral's RMSNorm: fp32 ``x * rsqrt(mean(x^2) + eps)``, cast back to
    the input dtype, times the weight."""

    x = hidden.float()
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return weight * x.to(hidden.dtype)


def stack_logits(stack: DecoderStack, context: ClosedLoopRunContext, tokens: torch.Tensor) -> torch.Tensor:
    """Logits ``[B,T,vocab]`` fp16 of ``tokens`` ``[B,T]`` with every layer's
    attention through ``context.codec``."""

    hidden = F.embedding(tokens, stack.embed)
    for layer, w in enumerate(stack.layers):
        attended = closed_loop_attention(rms_norm(hidden, w.input_norm, stack.rms_eps), w.attention,
                                         context.codec, layer, mode=context.mode, window=stack.window,
                                         rope_theta=stack.rope_theta, rate_records=context.rate_records)
        hidden = hidden + attended
        x = rms_norm(hidden, w.post_attention_norm, stack.rms_eps)
        hidden = hidden + F.linear(F.silu(F.linear(x, w.gate)) * F.linear(x, w.up), w.down)
    return F.linear(rms_norm(hidden, stack.final_norm, stack.rms_eps), stack.lm_head)


def causal_loss(logits: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """Mean next-token cross-entropy in fp32 (train_full_model_closed_loop_vq.py:359-364)."""

    return F.cross_entropy(logits[:, :-1].float().reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1),
                           reduction="mean")


def run_loss(stack: DecoderStack, context: ClosedLoopRunContext, tokens: torch.Tensor, *,
             mode: str) -> tuple[torch.Tensor, list[dict[str, Any]]]:
    """train_full_model_closed_loop_vq.py:367-377: reset the context, run
    the stack, return the causal loss and the forward's rate records."""

    context.reset(mode)
    loss = causal_loss(stack_logits(stack, context, tokens), tokens)
    return loss, list(context.rate_records)


def v_only_step(
    context: ClosedLoopRunContext,
    loss_fn,
    *,
    step: int,
    lr: float = 0.001,
    maximum_norm: float = 1.0,
) -> dict[str, Any]:
    """One step of train_mistral_v_only.py:143-153.

    ``loss_fn()`` returns ``(loss, rate_records)`` (``run_loss`` bound to a
    stack and its tokens).  ``step`` is the loop's 0-based index; the error
    texts count from 1 as the reference's do.  Returns the loss, the number
    of value tables whose gradient the clip scaled, and the clip record.
    """

    values: Sequence[torch.Tensor] = list(context.codec.value_tables)
    for table in values:  # optimizer.zero_grad(set_to_none=True)
        table.grad = None
    loss, rates = loss_fn()
    if rates or not bool(torch.isfinite(loss)):
        raise RuntimeError(f"nonfinite loss or unexpected rate at step {step + 1}")
    loss.backward()
    grads = [table.grad for table in values]
    if any(g is None for g in grads) or not bool(torch.stack([torch.isfinite(g).all() for g in grads]).all()):
        raise RuntimeError(f"nonfinite/missing V gradient at step {step + 1}")
    clipped = clip_codebook_gradients(context.codec, maximum_norm=maximum_norm, mode="per_layer_kv")
    clips = sum(bool(row["clip_activated"]) for row in clipped["per_group"] if row["kind"] == "value")
    sgd_step(values, lr=lr)
    return {"loss": float(loss.detach()), "clipped_value_layers": clips, "clip": clipped}
