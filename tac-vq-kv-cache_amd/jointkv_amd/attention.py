"""Attention consumers of the quantized cache: decode straight from a packed
uint8 code cache, and prefill over a chunk's quantized K̂/V̂.

The reference's LongBench decode loop (experiments_followup_mistral/
evaluate_mistral_longbench.py:29-124) keeps uint8 codes *and* a decoded fp16
4096-token workspace, re-applies RoPE to all visible keys every step, repeats
K/V across the GQA group and calls SDPA.  Here the cache holds only codes
(a ring buffer of ``capacity`` slots per (batch, kv head)), and one fused
kernel rebuilds K̂/V̂ from fp16 codewords, rotates K̂ at its absolute
position, and runs split-KV softmax attention for every query head of the
group.  The fp16 workspace, the RoPE pass over the window, ``repeat_kv`` and
the O(T) ``torch.cat`` appends disappear.
"""

from __future__ import annotations

import torch

from . import _ops

MISTRAL_WINDOW = 4096
MISTRAL_ROPE_THETA = 10000.0


def deploy_tables(tables: torch.Tensor, groups: int | None = None) -> torch.Tensor:
    """fp16 deployed codebooks ``[KVH*G,S,K,d]`` from fp32 masters.

    Accepts ``[H,S,K,D]`` (residual VQ, G=1), ``[H,G,S,K,d]`` (grouped
    residual) or ``[H,G,K,d]`` with ``groups`` given (grouped CQ, S=1).
    """

    if tables.ndim == 5:
        h, g, s, k, d = tables.shape
        flat = tables.reshape(h * g, s, k, d)
    elif tables.ndim == 4 and groups is not None:
        h, g, k, d = tables.shape
        flat = tables.reshape(h * g, 1, k, d)
    elif tables.ndim == 4:
        flat = tables
    else:
        raise ValueError("unsupported codebook geometry")
    return _ops.f32_to_f16(flat.contiguous())


def decode_attention(
    query: torch.Tensor,
    key_codes: torch.Tensor,
    value_codes: torch.Tensor,
    key_tables16: torch.Tensor,
    value_tables16: torch.Tensor,
    lengths: torch.Tensor,
    *,
    window: int = MISTRAL_WINDOW,
    rope_theta: float = MISTRAL_ROPE_THETA,
    max_length: int | None = None,
    key_new: torch.Tensor | None = None,
    value_new: torch.Tensor | None = None,
) -> torch.Tensor:
    """Attention output for one new token per sequence.

    ``query``: pre-RoPE ``[B,QH,1,D]`` or ``[B,QH,D]`` fp16.  ``key_codes``,
    ``value_codes``: ``[B,KVH,cap,G,S]`` (or ``[B,KVH,cap,G*S]``) uint8 with
    position p in slot ``p % cap``.  ``lengths[b]`` counts the cached tokens
    including the new one, so the query sits at position ``lengths[b]-1``
    and sees the last ``min(window, lengths[b])`` positions (the reference's
    ``LayerCache.visible``).  ``max_length`` (an upper bound of ``lengths``)
    avoids a device read.  With ``key_new``/``value_new`` (the raw
    ``[B,KVH,1,D]`` or ``[B,KVH,D]`` fp16 K/V of the token at position
    ``lengths[b]-1``) the launch first encodes that token into its ring slot
    (the codec call and ``LayerCache.append`` of
    evaluate_mistral_longbench.py:94-98, fused; group dim 8 caches).
    Returns ``[B,QH,1,D]`` (or ``[B,QH,D]``) fp16.
    """

    squeeze = query.ndim == 3
    q = query if squeeze else query.reshape(query.shape[0], query.shape[1], query.shape[-1])
    if key_codes.ndim == 4:
        groups = key_tables16.shape[0] // key_codes.shape[1]
        stages = key_codes.shape[-1] // groups
        key_codes = key_codes.unflatten(-1, (groups, stages))
        value_codes = value_codes.unflatten(-1, (groups, stages))
    if key_new is not None and key_new.ndim == 4:
        key_new = key_new.reshape(key_new.shape[0], key_new.shape[1], key_new.shape[-1])
    if value_new is not None and value_new.ndim == 4:
        value_new = value_new.reshape(value_new.shape[0], value_new.shape[1], value_new.shape[-1])
    out = _ops.decode_attention(
        q, key_codes, value_codes, key_tables16, value_tables16, lengths,
        window=window, rope_theta=rope_theta, max_length=max_length, key_new=key_new, value_new=value_new,
    )
    return out if squeeze else out.unsqueeze(2)


def decode_attention_window(
    query: torch.Tensor,
    key_window: torch.Tensor,
    value_window: torch.Tensor,
    lengths: torch.Tensor,
    *,
    window: int = MISTRAL_WINDOW,
    rope_theta: float = MISTRAL_ROPE_THETA,
    max_length: int | None = None,
) -> torch.Tensor:
    """:func:`decode_attention` over decoded fp16 K̂/V̂ instead of codes.

    The reference's own decode branch (evaluate_mistral_longbench.py:112-122)
    over ``LayerCache``'s decoded window (:44-70), for codecs whose codewords
    do not fit the packed-code kernel (full-vector R16/R32 tables: 1 MiB of
    fp16 codewords per kv head at 16 stages).  ``key_window``/``value_window``
    ``[B,KVH,cap,128]`` fp16 hold position p in slot ``p % cap`` (see
    :class:`DecodedWindowCache`); the rest is as in :func:`decode_attention`.
    """

    squeeze = query.ndim == 3
    q = query if squeeze else query.reshape(query.shape[0], query.shape[1], query.shape[-1])
    out = _ops.decode_attention_window(q, key_window, value_window, lengths, window=window,
                                       rope_theta=rope_theta, max_length=max_length)
    return out if squeeze else out.unsqueeze(2)


def _start_tensor(start_positions, batch: int, tokens: int, device) -> tuple[torch.Tensor, int]:
    """int32 [B] device starts and the largest position they reach."""

    if isinstance(start_positions, torch.Tensor):
        starts = start_positions.to(device=device, dtype=torch.int32).reshape(-1)
        if starts.numel() == 1 and batch != 1:
            starts = starts.expand(batch).contiguous()
        top = int(starts.max().item()) if batch else 0
    else:
        values = [int(start_positions)] * batch if isinstance(start_positions, int) else [int(x) for x in start_positions]
        starts = torch.tensor(values, dtype=torch.int32, device=device)
        top = max(values) if values else 0
    if starts.shape != (batch,):
        raise ValueError("start positions must be one per batch row")
    return starts, top + max(tokens, 1) - 1


def prefill_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    start_positions=0,
    *,
    window: int = MISTRAL_WINDOW,
    rope_theta: float = MISTRAL_ROPE_THETA,
) -> torch.Tensor:
    """Attention of a prefill chunk over its own quantized K̂/V̂.

    The prefill branch of evaluate_mistral_longbench.py:101-111 (training
    twin train_full_model_closed_loop_vq.py:277-304): RoPE of ``query``
    ``[B,QH,T,128]`` and ``key`` ``[B,KVH,T,128]`` (fp16, pre-RoPE, e.g. the
    codec's reconstructions) at positions ``start + t``, ``repeat_kv``, and
    SDPA with the causal mask and Mistral's ``window``-token sliding window.
    ``start_positions``: an int, a sequence of B ints or an int32 tensor.
    Returns ``[B,QH,T,128]`` fp16.
    """

    batch, _qh, tokens, _d = map(int, query.shape)
    starts, top = _start_tensor(start_positions, batch, tokens, query.device)
    if torch.is_grad_enabled() and (query.requires_grad or key.requires_grad or value.requires_grad):
        return _PrefillAttention.apply(query, key, value, starts, window, rope_theta, top)
    return _ops.prefill_attention(query, key, value, starts, window=window, rope_theta=rope_theta,
                                  max_position=top)


class _PrefillAttention(torch.autograd.Function):
    """Prefill attention with a HIP backward: the forward keeps each row's
    log-sum-exp; the backward recomputes P from it.  Only the value is
    needed: dV̂ = Pᵀ dO summed over the GQA group (the V-only step).  Query
    or key too: the full backward (dS = P (dO V̂ᵀ - rowsum(dO O)), dQ = dS K̂,
    dK̂ = dSᵀ Q, through the rotary's transpose)."""

    @staticmethod
    def forward(ctx, query, key, value, starts, window, rope_theta, top):
        batch, qheads, tokens, _d = map(int, query.shape)
        lse = torch.empty((batch, qheads, tokens), dtype=torch.float32, device=query.device)
        out = _ops.prefill_attention(query, key, value, starts, window=window, rope_theta=rope_theta,
                                     max_position=top, lse=lse)
        ctx.save_for_backward(query, key, value, out, lse, starts)
        ctx.params = (window, rope_theta, top)
        return out

    @staticmethod
    def backward(ctx, d_out):
        query, key, value, out, lse, starts = ctx.saved_tensors
        window, rope_theta, top = ctx.params
        need_q, need_k, need_v = ctx.needs_input_grad[:3]
        d_out = d_out.to(torch.float16)
        if need_q or need_k:
            dq, dk, dv = _ops.prefill_attention_backward(
                query, key, value, out, d_out, lse, starts, window=window, rope_theta=rope_theta,
                max_position=top, need=(need_q, need_k, need_v))
        else:
            dq = dk = None
            dv = _ops.prefill_attention_value_grad(query, key, d_out, lse, starts, window=window,
                                                   rope_theta=rope_theta, max_position=top)
        # each input's dtype, as SDPA's backward returns it (fp32 sums, one rounding)
        return (dq.to(query.dtype) if dq is not None else None,
                dk.to(key.dtype) if dk is not None else None,
                dv.to(value.dtype) if (dv is not None and need_v) else None,
                None, None, None, None)


def prefill_attention_from_codes(
    query: torch.Tensor,
    key_codes: torch.Tensor,
    value_codes: torch.Tensor,
    key_tables16: torch.Tensor,
    value_tables16: torch.Tensor,
    start_positions=0,
    *,
    window: int = MISTRAL_WINDOW,
    rope_theta: float = MISTRAL_ROPE_THETA,
    fused: bool = False,
) -> torch.Tensor:
    """:func:`prefill_attention` for a chunk given as uint8 codes.

    ``key_codes``/``value_codes`` ``[B,KVH,T,G,S]`` and fp16 deployed tables
    ``[KVH*G,S,K,d]``; K̂/V̂ are the codec's reconstruction (fp16 of the fp32
    stage sum).  By default K̂/V̂ are decoded once into fp16 buffers and then
    attended.  ``fused=True`` (GSRQ geometries: 16 groups of 8 dims, 256
    codewords, one or two stages) rebuilds each K̂/V̂ tile inside the
    attention kernel as it loads it, so no K̂/V̂ buffer exists; every query
    block then rebuilds the tiles it reads, which makes it the slower of the
    two (about even at 128-token chunks, 1.45x at 2048).  Both give the same
    bits.
    """

    if fused:
        if not _ops.prefill_codes_supported(key_codes, key_tables16):
            raise ValueError("the fused prefill needs [B,KVH,T,16,S<=2] codes and [KVH*16,S,256,8] tables")
        batch, _qh, tokens, _d = map(int, query.shape)
        starts, top = _start_tensor(start_positions, batch, tokens, query.device)
        return _ops.prefill_attention_codes(query, key_codes, value_codes, key_tables16, value_tables16, starts,
                                            window=window, rope_theta=rope_theta, max_position=top)
    stages = int(key_codes.shape[-1])
    khat = _ops.rvq_decode(key_codes, key_tables16, depth=stages, dtype=torch.float16)
    vhat = _ops.rvq_decode(value_codes, value_tables16, depth=stages, dtype=torch.float16)
    return prefill_attention(query, khat, vhat, start_positions, window=window, rope_theta=rope_theta)


class PackedCodeCache:
    """Per-layer uint8 code cache for batched decode (ring buffer).

    Replaces ``LayerCache`` (evaluate_mistral_longbench.py:29-78) for the
    quantized path: it stores K and V codes only, appends in O(new tokens)
    into slot ``position % capacity``, and tracks per-sequence lengths.
    """

    def __init__(
        self,
        batch: int,
        kv_heads: int,
        groups: int,
        stages: int,
        *,
        capacity: int = MISTRAL_WINDOW,
        device: torch.device | str = "cuda",
    ) -> None:
        if min(batch, kv_heads, groups, stages, capacity) <= 0:
            raise ValueError("invalid code-cache geometry")
        shape = (batch, kv_heads, capacity, groups, stages)
        self.key = torch.zeros(shape, dtype=torch.uint8, device=device)
        self.value = torch.zeros(shape, dtype=torch.uint8, device=device)
        self.lengths = torch.zeros(batch, dtype=torch.int32, device=device)
        self.capacity = capacity
        self._host_length = 0

    @property
    def length(self) -> int:
        return self._host_length

    def append(self, key_codes: torch.Tensor, value_codes: torch.Tensor) -> None:
        """Append ``[B,KVH,T,G,S]`` codes for T new positions (all sequences)."""

        if key_codes.shape != value_codes.shape or key_codes.dtype != torch.uint8:
            raise ValueError("key/value codes differ")
        new = int(key_codes.shape[2])
        if new > self.capacity:
            key_codes = key_codes[:, :, -self.capacity :]
            value_codes = value_codes[:, :, -self.capacity :]
            self._host_length += new - self.capacity
            new = self.capacity
        start = self._host_length % self.capacity
        first = min(new, self.capacity - start)
        self.key[:, :, start : start + first] = key_codes[:, :, :first]
        self.value[:, :, start : start + first] = value_codes[:, :, :first]
        if first < new:
            self.key[:, :, : new - first] = key_codes[:, :, first:]
            self.value[:, :, : new - first] = value_codes[:, :, first:]
        self._host_length += new
        self.lengths.fill_(self._host_length)

    def encode_append(self, key: torch.Tensor, value: torch.Tensor, key_tables: torch.Tensor,
                      value_tables: torch.Tensor, *, group_dim: int) -> None:
        """Encode one new token per sequence (``key``/``value`` ``[B,KVH,1,G*d]``
        fp16, fp32 masters ``[KVH*G,S,K,d]``) straight into the next slot.

        The codes the codec would hand to ``LayerCache.append``
        (evaluate_mistral_longbench.py:94-98) land in the ring buffer without
        an intermediate tensor or copy.
        """

        if key.shape[2] != 1 or value.shape[2] != 1:
            raise ValueError("encode_append takes one token per sequence")
        slot = self._host_length % self.capacity
        groups = self.key.shape[3]
        # K and V in one launch (one token per sequence is latency-bound)
        _ops.rvq_encode_kv(key, value, key_tables, value_tables, groups=groups, group_dim=group_dim, exits=(),
                           key_codes_out=self.key[:, :, slot : slot + 1],
                           value_codes_out=self.value[:, :, slot : slot + 1])
        self._host_length += 1
        self.lengths.fill_(self._host_length)

    def attend_append(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                      key_tables16: torch.Tensor, value_tables16: torch.Tensor, *,
                      window: int = MISTRAL_WINDOW, rope_theta: float = MISTRAL_ROPE_THETA) -> torch.Tensor:
        """One decode step in one launch: encode the new token's raw K/V
        (``[B,KVH,1,128]`` fp16) with the fp16 deployed tables
        ``[KVH*G,S,K,8]`` into the next slot and attend over the window
        (evaluate_mistral_longbench.py:94-122).  Returns ``[B,QH,1,128]``
        (or ``[B,QH,128]`` for a 3-D query)."""

        if (key.ndim == 4 and key.shape[2] != 1) or (value.ndim == 4 and value.shape[2] != 1):
            raise ValueError("attend_append takes one token per sequence")
        # the cache counts the new token only once the launch that writes its
        # codes has been accepted: a refused geometry (the fused append serves
        # 16 groups of 8 dims, S <= 2) leaves length and lengths unchanged, so
        # a caller can fall back to encode_append + decode_attention
        new_length = self._host_length + 1
        self.lengths.fill_(new_length)
        try:
            out = decode_attention(query, self.key, self.value, key_tables16, value_tables16, self.lengths,
                                   window=window, rope_theta=rope_theta, max_length=new_length,
                                   key_new=key, value_new=value)
        except BaseException:
            self.lengths.fill_(self._host_length)
            raise
        self._host_length = new_length
        return out

    def payload_bytes(self) -> int:
        visible = min(self._host_length, self.capacity)
        per_slot = self.key.shape[3] * self.key.shape[4]
        return 2 * self.key.shape[0] * self.key.shape[1] * visible * per_slot


class DecodedWindowCache:
    """Per-layer cache that keeps the decoded fp16 K̂/V̂ window, as the
    reference's ``LayerCache`` does (evaluate_mistral_longbench.py:29-78,
    its "declared evaluation acceleration workspace" :57), plus the uint8
    code payload.

    Both live in ring buffers (slot ``position % capacity``) instead of
    ``torch.cat`` + slicing, so an append costs O(new tokens).  Use it for
    codecs the packed-code kernel does not serve at speed (full-vector
    R16/R32 tables); attend with :meth:`attention`.
    """

    def __init__(
        self,
        batch: int,
        kv_heads: int,
        groups: int,
        stages: int,
        *,
        capacity: int = MISTRAL_WINDOW,
        head_dim: int = 128,
        device: torch.device | str = "cuda",
    ) -> None:
        if min(batch, kv_heads, groups, stages, capacity) <= 0 or head_dim != 128:
            raise ValueError("invalid decoded-window cache geometry")
        self.codes = PackedCodeCache(batch, kv_heads, groups, stages, capacity=capacity, device=device)
        shape = (batch, kv_heads, capacity, head_dim)
        self.decoded_key = torch.zeros(shape, dtype=torch.float16, device=device)
        self.decoded_value = torch.zeros(shape, dtype=torch.float16, device=device)
        self.capacity = capacity

    @property
    def length(self) -> int:
        return self.codes.length

    @property
    def lengths(self) -> torch.Tensor:
        return self.codes.lengths

    def append(self, key_codes: torch.Tensor, value_codes: torch.Tensor, decoded_key: torch.Tensor,
               decoded_value: torch.Tensor) -> None:
        """``LayerCache.append`` (:44-60): codes ``[B,KVH,T,G,S]`` and the
        codec's fp16 reconstructions ``[B,KVH,T,128]`` for T new positions."""

        new = int(key_codes.shape[2])
        if decoded_key.shape[2] != new or decoded_value.shape[2] != new:
            raise ValueError("codes and decoded rows cover different tokens")
        if decoded_key.dtype != torch.float16 or decoded_value.dtype != torch.float16:
            raise ValueError("decoded rows must be fp16")
        start_length = self.codes.length
        self.codes.append(key_codes, value_codes)
        if new > self.capacity:
            decoded_key = decoded_key[:, :, -self.capacity :]
            decoded_value = decoded_value[:, :, -self.capacity :]
            start_length += new - self.capacity
            new = self.capacity
        start = start_length % self.capacity
        first = min(new, self.capacity - start)
        self.decoded_key[:, :, start : start + first] = decoded_key[:, :, :first]
        self.decoded_value[:, :, start : start + first] = decoded_value[:, :, :first]
        if first < new:
            self.decoded_key[:, :, : new - first] = decoded_key[:, :, first:]
            self.decoded_value[:, :, : new - first] = decoded_value[:, :, first:]

    def encode_append(self, key: torch.Tensor, value: torch.Tensor, key_tables: torch.Tensor,
                      value_tables: torch.Tensor, *, group_dim: int) -> None:
        """Run the codec on one new token per sequence (``[B,KVH,1,128]``
        fp16, fp32 masters ``[KVH*G,S,K,d]``): its codes go to the payload
        ring and its full-depth reconstructions to the decoded window, as
        evaluate_mistral_longbench.py:94-98 hands both to ``LayerCache``."""

        if key.shape[2] != 1 or value.shape[2] != 1:
            raise ValueError("encode_append takes one token per sequence")
        groups, stages = self.codes.key.shape[3], self.codes.key.shape[4]
        slot = self.codes.length % self.capacity
        recon_k, _, recon_v, _ = _ops.rvq_encode_kv(
            key, value, key_tables, value_tables, groups=groups, group_dim=group_dim, exits=(stages,),
            key_codes_out=self.codes.key[:, :, slot : slot + 1],
            value_codes_out=self.codes.value[:, :, slot : slot + 1])
        self.decoded_key[:, :, slot : slot + 1] = recon_k[0]
        self.decoded_value[:, :, slot : slot + 1] = recon_v[0]
        self.codes._host_length += 1
        self.codes.lengths.fill_(self.codes._host_length)

    def attention(self, query: torch.Tensor, *, window: int | None = None,
                  rope_theta: float = MISTRAL_ROPE_THETA) -> torch.Tensor:
        """Decode attention of ``query`` ``[B,QH,1,128]`` over the window."""

        return decode_attention_window(query, self.decoded_key, self.decoded_value, self.codes.lengths,
                                       window=self.capacity if window is None else window,
                                       rope_theta=rope_theta, max_length=self.codes.length)

    def payload_bytes(self) -> int:
        return self.codes.payload_bytes()

    def decode_workspace_bytes(self) -> int:
        visible = min(self.codes.length, self.capacity)
        return 2 * self.decoded_key.shape[0] * self.decoded_key.shape[1] * visible * self.decoded_key.shape[3] * 2
