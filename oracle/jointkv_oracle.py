"""CPU oracle for the jointkv hard residual-quantization hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker or as the timed CPU baseline.  The product (``jointkv_amd``) never
calls it.

Each function restates, with eager PyTorch ops on the CPU, the arithmetic of
the reference operator it names (same fp32 distance formula, same argmin tie
rule, same fp16 deploy round trip, same stage order, same autograd graph), so
its outputs are what the reference computes on the same inputs.  The
reference itself is pure Python/PyTorch; it was read, not run.

Pins (see tests/test_oracle_*.py):
  * nearest search and greedy residual stages: fp64 exhaustive brute force
    in ``oracle/c/vq_bruteforce.c`` (codes equal wherever the fp64 margin
    clears fp32 noise), plus the reference's own relational tests
    (exits equal the decode of the codes; fp16-persistent codewords).
  * straight-through gradient: the closed form
    grad[h,s,k] = sum_{n: code[n,s]=k} dL/dX̂[n] checked by brute force in C,
    and the reference's 1-D known answer (table [0,1,10,20], state 0.1:
    gradient exactly 1.0 on word 0, zero elsewhere).
  * clip: the reference's exact numeric expectations
    (tests/test_pure_uniform16_closed_loop_vq.py:53-138).
  * decode/prefill attention: fp64 textbook softmax attention with the
    rotate-half RoPE; HF transformers' fp16 rotary arithmetic itself is
    third-party (transformers 4.45.1, not vendored) and is restated from its
    published definition.
"""

from __future__ import annotations

import math
from collections.abc import Sequence

import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# Nearest search and residual VQ


def nearest_indices(states: torch.Tensor, table: torch.Tensor, *, token_chunk_size: int) -> torch.Tensor:
    """argmin_k |r|^2 + |c_k|^2 - 2 r.c_k in fp32, chunked over rows.

    Follows src/jointkv/closed_loop_vq.py:52-76 (first index on ties).
    states [H,N,D], table [H,K,D] -> int64 [H,N].
    """

    norms = table.square().sum(dim=-1)
    out = []
    for start in range(0, states.shape[1], token_chunk_size):
        rows = states[:, start : start + token_chunk_size]
        dist = rows.square().sum(dim=-1, keepdim=True) + norms[:, None, :] - 2.0 * torch.bmm(
            rows, table.transpose(-1, -2)
        )
        out.append(dist.argmin(dim=-1))
    return torch.cat(out, dim=1)


def distances_top2(states: torch.Tensor, table: torch.Tensor, *, token_chunk_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Best and second-best fp32 distances with the same formula (for margins)."""

    norms = table.square().sum(dim=-1)
    best, second = [], []
    for start in range(0, states.shape[1], token_chunk_size):
        rows = states[:, start : start + token_chunk_size]
        dist = rows.square().sum(dim=-1, keepdim=True) + norms[:, None, :] - 2.0 * torch.bmm(
            rows, table.transpose(-1, -2)
        )
        k = min(2, dist.shape[-1])
        vals = dist.topk(k, dim=-1, largest=False).values
        best.append(vals[..., 0])
        second.append(vals[..., -1] if k == 2 else torch.full_like(vals[..., 0], float("inf")))
    return torch.cat(best, dim=1), torch.cat(second, dim=1)


def hard_residual_vq_exits(
    states: torch.Tensor,
    tables: torch.Tensor,
    *,
    prefixes: Sequence[int],
    assignment_whiteners: torch.Tensor | None = None,
    token_chunk_size: int = 1024,
    straight_through_states: bool = True,
    return_margins: bool = False,
    forced_codes: torch.Tensor | None = None,
):
    """Greedy residual VQ exactly as src/jointkv/closed_loop_vq.py:235-410.

    states [B,H,T,D], tables [H,S,K,D] (fp32 masters).  The search and the
    reconstruction use ``tables.half().float()`` (:298); with a whitener the
    search runs on W x and W c and subtracts whitened codewords (:312-330,
    :384-390).  ``decoded`` accumulates fp32 codewords in stage order (:381)
    and each exit is cast once to states.dtype (:396-402), plus the identity
    straight-through edge (:408).  Autograd reaches the fp32 masters through
    ``torch.gather`` (:376-381).  With ``return_margins`` also returns the
    best and second-best fp32 search distances per (B,H,T,S).

    ``forced_codes`` [B,H,T,S] (test use: another implementation's choices)
    makes every stage reconstruct and subtract the forced codeword instead
    of its own pick, so that a near-tie resolved the other way does not
    change the rest of the chain; the returned codes and margins are still
    this search's own, made on the forced chain's residuals, which is what
    judging the other implementation's choice stage by stage needs.
    """

    batch, heads, tokens, dim = map(int, states.shape)
    stages = int(tables.shape[1])
    requested = tuple(sorted(set(int(p) for p in prefixes)))
    x = states.detach().float()
    raw = x.permute(1, 0, 2, 3).reshape(heads, batch * tokens, dim).contiguous().clone()
    deployed = tables + (tables.half().float() - tables).detach()
    frozen = deployed.detach().float()
    search_rows = raw
    search_tables = frozen
    if assignment_whiteners is not None:
        w = assignment_whiteners.detach().float()
        search_rows = (
            torch.einsum("hde,bhte->bhtd", w, x).permute(1, 0, 2, 3).reshape(heads, batch * tokens, dim).contiguous()
        )
        search_tables = torch.einsum("hrke,hde->hrkd", frozen, w)
    decoded = torch.zeros((heads, batch * tokens, dim), dtype=torch.float32)
    codes = torch.empty((batch, heads, tokens, stages), dtype=torch.uint8)
    d1 = torch.empty((batch, heads, tokens, stages), dtype=torch.float32)
    d2 = torch.empty_like(d1)
    outputs = {}
    for s in range(stages):
        table_s = search_tables[:, s]
        with torch.no_grad():
            idx = own = nearest_indices(search_rows, table_s, token_chunk_size=token_chunk_size)
            if return_margins:
                b1, b2 = distances_top2(search_rows, table_s, token_chunk_size=token_chunk_size)
                d1[..., s] = b1.reshape(heads, batch, tokens).permute(1, 0, 2)
                d2[..., s] = b2.reshape(heads, batch, tokens).permute(1, 0, 2)
            if forced_codes is not None:
                idx = forced_codes[..., s].permute(1, 0, 2).reshape(heads, batch * tokens).long()
        chosen = torch.gather(deployed[:, s].float(), 1, idx[..., None].expand(-1, -1, dim))
        decoded = decoded + chosen
        with torch.no_grad():
            raw.sub_(chosen.detach())
            if assignment_whiteners is not None:
                search_rows.sub_(torch.gather(table_s, 1, idx[..., None].expand(-1, -1, dim)))
            codes[..., s] = own.reshape(heads, batch, tokens).permute(1, 0, 2).to(torch.uint8)
        if s + 1 in requested:
            out = decoded.reshape(heads, batch, tokens, dim).permute(1, 0, 2, 3).contiguous().to(states.dtype)
            if straight_through_states:
                out = out + (states - states.detach())
            outputs[s + 1] = out
    if return_margins:
        return outputs, codes, d1, d2
    return outputs, codes


def grouped_residual_vq(
    states: torch.Tensor,
    tables: torch.Tensor,
    *,
    prefixes: Sequence[int],
    token_chunk_size: int = 1024,
    straight_through_states: bool = True,
    return_margins: bool = False,
    forced_codes: torch.Tensor | None = None,
):
    """Grouped residual VQ via the reference's own call on folded heads.

    states [B,H,T,G*d], tables [H,G,S,K,d]: fold (head, group) into the head
    axis, call :func:`hard_residual_vq_exits` (the reference operator), and
    unfold: codes [B,H,T,G,S], exits [B,H,T,G*d].  ``forced_codes``
    [B,H,T,G,S]: as in :func:`hard_residual_vq_exits`.
    """

    batch, heads, tokens, dim = map(int, states.shape)
    _h, groups, stages, clusters, d = map(int, tables.shape)
    folded = states.reshape(batch, heads, tokens, groups, d).permute(0, 1, 3, 2, 4).reshape(
        batch, heads * groups, tokens, d
    )
    res = hard_residual_vq_exits(
        folded,
        tables.reshape(heads * groups, stages, clusters, d),
        prefixes=prefixes,
        token_chunk_size=token_chunk_size,
        straight_through_states=straight_through_states,
        return_margins=return_margins,
        forced_codes=None if forced_codes is None else forced_codes.permute(0, 1, 3, 2, 4).reshape(
            batch, heads * groups, tokens, stages),
    )
    outputs, codes = res[0], res[1]

    def unfold_rows(t):
        return t.reshape(batch, heads, groups, tokens, -1).permute(0, 1, 3, 2, 4)

    out = {k: unfold_rows(v).reshape(batch, heads, tokens, dim) for k, v in outputs.items()}
    codes_u = unfold_rows(codes).contiguous()
    if return_margins:
        return out, codes_u, unfold_rows(res[2]).contiguous(), unfold_rows(res[3]).contiguous()
    return out, codes_u


def hard_grouped_cq(
    states: torch.Tensor,
    codebooks: torch.Tensor,
    *,
    selector_whiteners: torch.Tensor | None = None,
    token_chunk_size: int = 64,
    straight_through_states: bool = True,
    return_margins: bool = False,
):
    """Grouped CQ exactly as src/jointkv/cq_tac.py:33-114.

    states [B,H,T,D], codebooks [H,G,K,S] -> (recon [B,H,T,D], codes [B,H,T,G]).
    """

    batch, heads, tokens, dim = map(int, states.shape)
    _h, groups, clusters, sub = map(int, codebooks.shape)
    problems, rows_n = heads * groups, batch * tokens
    raw = (
        states.detach().float().permute(1, 0, 2, 3).reshape(heads, rows_n, groups, sub)
        .permute(0, 2, 1, 3).reshape(problems, rows_n, sub).contiguous()
    )
    deployed = codebooks + (codebooks.half().float() - codebooks).detach()
    search_tables = deployed.detach().float().reshape(problems, clusters, sub)
    search_rows = raw
    if selector_whiteners is not None:
        f = selector_whiteners.detach().float().reshape(problems, sub, sub)
        search_rows = torch.bmm(raw, f.transpose(1, 2))
        search_tables = torch.bmm(search_tables, f.transpose(1, 2))
    norms = search_tables.square().sum(-1).unsqueeze(1)
    idx = torch.empty(problems, rows_n, dtype=torch.long)
    b1 = torch.empty(problems, rows_n)
    b2 = torch.empty(problems, rows_n)
    for start in range(0, rows_n, token_chunk_size):
        stop = min(start + token_chunk_size, rows_n)
        cur = search_rows[:, start:stop]
        dist = cur.square().sum(-1, keepdim=True) + norms - 2.0 * torch.bmm(cur, search_tables.transpose(1, 2))
        idx[:, start:stop] = dist.argmin(-1)
        if return_margins:
            k = min(2, clusters)
            vals = dist.topk(k, dim=-1, largest=False).values
            b1[:, start:stop] = vals[..., 0]
            b2[:, start:stop] = vals[..., -1] if k == 2 else float("inf")
    live = deployed.reshape(problems, clusters, sub)
    chosen = torch.gather(live, 1, idx[..., None].expand(-1, -1, sub))
    out = (
        chosen.reshape(heads, groups, batch, tokens, sub).permute(2, 0, 3, 1, 4)
        .reshape(batch, heads, tokens, dim).to(states.dtype)
    )
    if straight_through_states:
        out = out + (states - states.detach())

    def shape_rows(t):
        return t.reshape(heads, groups, batch, tokens).permute(2, 0, 3, 1).contiguous()

    codes = shape_rows(idx).to(torch.uint8)
    if return_margins:
        return out, codes, shape_rows(b1), shape_rows(b2)
    return out, codes


def frozen_decode(codes: torch.Tensor, tables: torch.Tensor, depth: int, dtype: torch.dtype) -> torch.Tensor:
    """fp16-deployed decode of given codes: codes [B,H,T,G,S], tables [H*G,S,K,d].

    Same arithmetic as frozen_assignment_u16_reconstruction
    (experiments/train_pure_uniform16_closed_loop_vq.py:395-442): fp32 sum of
    fp16 round-tripped words in stage order, one cast at the end.
    """

    batch, heads, tokens, groups, stages = map(int, codes.shape)
    problems, _s, clusters, d = map(int, tables.shape)
    deployed = tables.detach().half().float()
    flat = codes.long().permute(1, 3, 0, 2, 4).reshape(heads * groups, batch * tokens, stages)
    acc = torch.zeros(problems, batch * tokens, d)
    for s in range(depth):
        acc = acc + torch.gather(deployed[:, s], 1, flat[..., s, None].expand(-1, -1, d))
    return acc.reshape(heads, groups, batch, tokens, d).permute(2, 0, 3, 1, 4).reshape(
        batch, heads, tokens, groups * d
    ).to(dtype)


def table_gradient(
    grads: Sequence[torch.Tensor],
    exits: Sequence[int],
    codes: torch.Tensor,
    table_shape,
    accumulate: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Closed form of the gather backward: codes [B,H,T,G,S], grads [B,H,T,G*d].

    grad[p,s,k,:] = sum over rows with code[.., g, s] = k of
    sum_{exits e: depth_e > s} fp32(grads_e[.., g*d:(g+1)*d]).
    This is what autograd computes for closed_loop_vq.py:376-381 / cq_tac.py:98-99.
    ``accumulate=torch.float64`` sums in fp64 and returns fp64: for fp16
    gradients at test sizes that sum is exact, so ``.float()`` of it is the
    correctly rounded fp32 result.
    """

    batch, heads, tokens, groups, stages = map(int, codes.shape)
    problems, _s, clusters, d = map(int, table_shape)
    out = torch.zeros(table_shape, dtype=accumulate)
    flat_codes = codes.long().permute(1, 3, 0, 2, 4).reshape(problems, batch * tokens, stages)
    for s in range(stages):
        g = None
        for grad, depth in zip(grads, exits):
            if depth > s:
                gf = grad.to(accumulate).reshape(batch, heads, tokens, groups, d).permute(1, 3, 0, 2, 4).reshape(
                    problems, batch * tokens, d
                )
                g = gf if g is None else g + gf
        if g is None:
            continue
        out[:, s].scatter_add_(1, flat_codes[..., s, None].expand(-1, -1, d), g)
    return out


# ---------------------------------------------------------------------------
# Gradient clipping (experiments/train_pure_uniform16_closed_loop_vq.py:1151-1304)


def clip_codebook_gradients(key_tables, value_tables, *, maximum_norm: float, mode: str) -> dict:
    """Restatement with torch.nn.utils.clip_grad_norm_ on CPU parameters."""

    if not math.isfinite(maximum_norm) or maximum_norm <= 0:
        raise ValueError("gradient cap must be finite and positive")
    groups = [(layer, kind, p) for kind, tabs in (("key", key_tables), ("value", value_tables)) for layer, p in enumerate(tabs)]

    def norm(p):
        return 0.0 if p.grad is None else float(torch.linalg.vector_norm(p.grad.detach().float()))

    if mode == "global":
        params = [p for _l, _k, p in groups if p.requires_grad]
        if not params:
            raise RuntimeError("gradient clipping received no trainable codebooks")
        before = float(torch.nn.utils.clip_grad_norm_(params, maximum_norm))
        return {
            "mode": mode,
            "group_count": len(groups),
            "trainable_group_count": len(params),
            "total_norm_before_clip": before,
            "total_norm_after_clip": min(before, maximum_norm),
            "global_scale": min(1.0, maximum_norm / (before + 1e-12)),
            "per_group": None,
        }
    if mode not in {"per_layer_kv", "key_global_value_per_layer"}:
        raise ValueError(f"unknown gradient clip mode: {mode}")
    rows = []
    if mode == "key_global_value_per_layer":
        keys = [g for g in groups if g[1] == "key"]
        key_before = {layer: norm(p) for layer, _k, p in keys}
        key_total = math.sqrt(sum(v * v for v in key_before.values()))
        key_params = [p for _l, _k, p in keys if p.requires_grad]
        if key_params:
            torch.nn.utils.clip_grad_norm_(key_params, maximum_norm)
        for layer, kind, p in keys:
            b, a = key_before[layer], norm(p)
            rows.append({"layer": layer, "kind": kind, "norm_before_clip": b, "norm_after_clip": a,
                         "scale": 1.0 if b == 0.0 else a / b, "clip_activated": key_total > maximum_norm})
        rest = [g for g in groups if g[1] == "value"]
    else:
        rest = groups
        key_total = None
    for layer, kind, p in rest:
        if p.grad is None:
            b = a = 0.0
        else:
            b = norm(p)
            torch.nn.utils.clip_grad_norm_([p], maximum_norm)
            a = norm(p)
        rows.append({"layer": layer, "kind": kind, "norm_before_clip": b, "norm_after_clip": a,
                     "scale": 1.0 if b == 0.0 else a / b, "clip_activated": b > maximum_norm})
    out = {
        "mode": mode,
        "total_norm_before_clip": math.sqrt(sum(r["norm_before_clip"] ** 2 for r in rows)),
        "total_norm_after_clip": math.sqrt(sum(r["norm_after_clip"] ** 2 for r in rows)),
        "per_group": rows,
    }
    if key_total is not None:
        out["key_global_norm_before_clip"] = key_total
    return out


# ---------------------------------------------------------------------------
# Attention consumers


def rotary_cos_sin(positions: torch.Tensor, head_dim: int, theta: float, dtype=torch.float16):
    """Rotary tables as the HF Mistral/Llama rotary module builds them.

    inv_freq = 1/theta^(arange(0,D,2)/D) in fp32; angle = position*inv_freq
    in fp32; emb = cat(freqs, freqs); cos/sin in fp32 cast to ``dtype``
    (transformers 4.45.1, third-party: restated from its published code).
    """

    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """(x * cos) + (rotate_half(x) * sin) in x.dtype (HF apply_rotary_pos_emb)."""

    return (x * cos) + (rotate_half(x) * sin)


def decode_attention(
    q: torch.Tensor,
    key_hat: torch.Tensor,
    value_hat: torch.Tensor,
    query_position: int,
    key_positions: torch.Tensor,
    *,
    theta: float = 10000.0,
) -> torch.Tensor:
    """One decode step as evaluate_mistral_longbench.py:112-122.

    q [B,QH,1,D] fp16 pre-RoPE; key_hat/value_hat [B,KVH,Tvis,D] fp16
    (decoded, pre-RoPE); RoPE(q) at query_position, RoPE(K̂) at
    key_positions, repeat_kv, SDPA without mask.  Returns [B,QH,1,D] fp16.
    """

    head_dim = q.shape[-1]
    qc, qs = rotary_cos_sin(torch.tensor([query_position]), head_dim, theta)
    kc, ks = rotary_cos_sin(key_positions, head_dim, theta)
    qr = apply_rotary(q, qc[None, None], qs[None, None])
    kr = apply_rotary(key_hat, kc[None, None], ks[None, None])
    groups = q.shape[1] // key_hat.shape[1]
    kr = kr.repeat_interleave(groups, dim=1)
    vr = value_hat.repeat_interleave(groups, dim=1)
    # fp32 math on the fp16-rounded operands; output rounded to fp16
    out = F.scaled_dot_product_attention(qr.float(), kr.float(), vr.float(), attn_mask=None, dropout_p=0.0)
    return out.to(torch.float16)


def sliding_causal_mask(tokens: int, window: int) -> torch.Tensor:
    """[T,T] bool: query t sees key s iff s <= t and t - s < window.

    The causal mask with Mistral's sliding window (HF transformers 4.45.1
    Mistral attention mask, third-party; restated) for a chunk whose
    positions are consecutive.
    """

    t = torch.arange(tokens)
    diff = t[:, None] - t[None, :]
    return (diff >= 0) & (diff < window)


def prefill_attention(
    q: torch.Tensor,
    key_hat: torch.Tensor,
    value_hat: torch.Tensor,
    start_positions: Sequence[int],
    *,
    window: int = 4096,
    theta: float = 10000.0,
) -> torch.Tensor:
    """The prefill branch of evaluate_mistral_longbench.py:101-111 (and its
    training twin train_full_model_closed_loop_vq.py:277-304).

    q [B,QH,T,D] fp16 pre-RoPE; key_hat/value_hat [B,KVH,T,D] fp16 (the
    chunk's quantized K/V, pre-RoPE).  Positions of batch row b are
    start_positions[b] + t.  RoPE(q), RoPE(K̂) in fp16, repeat_kv, SDPA with
    the causal sliding-window mask in fp32 on the fp16 operands; output fp16
    [B,QH,T,D].
    """

    batch, _qh, tokens, head_dim = map(int, q.shape)
    groups = q.shape[1] // key_hat.shape[1]
    mask = sliding_causal_mask(tokens, window)
    outs = []
    for b in range(batch):
        pos = torch.arange(tokens) + int(start_positions[b])
        c, s = rotary_cos_sin(pos, head_dim, theta)
        qr = apply_rotary(q[b : b + 1], c[None, None], s[None, None])
        kr = apply_rotary(key_hat[b : b + 1], c[None, None], s[None, None])
        kr = kr.repeat_interleave(groups, dim=1)
        vr = value_hat[b : b + 1].repeat_interleave(groups, dim=1)
        out = F.scaled_dot_product_attention(qr.float(), kr.float(), vr.float(), attn_mask=mask, dropout_p=0.0)
        outs.append(out.to(torch.float16))
    return torch.cat(outs, dim=0)


def _rotated_chunk(q, key_hat, start, window, theta, b):
    tokens, head_dim = int(q.shape[2]), int(q.shape[3])
    pos = torch.arange(tokens) + int(start)
    c, s = rotary_cos_sin(pos, head_dim, theta)
    qr = apply_rotary(q[b : b + 1], c[None, None], s[None, None])
    kr = apply_rotary(key_hat[b : b + 1], c[None, None], s[None, None])
    return qr, kr.repeat_interleave(q.shape[1] // key_hat.shape[1], dim=1), sliding_causal_mask(tokens, window)


def prefill_lse(
    q: torch.Tensor,
    key_hat: torch.Tensor,
    start_positions: Sequence[int],
    *,
    window: int = 4096,
    theta: float = 10000.0,
) -> torch.Tensor:
    """Each row's natural log-sum-exp of its visible scores
    RoPE(q).RoPE(K̂)/sqrt(D), fp32 on the fp16-rotated operands: the row
    normaliser of :func:`prefill_attention`'s softmax.  [B,QH,T] fp32."""

    out = []
    for b in range(q.shape[0]):
        qr, kr, mask = _rotated_chunk(q, key_hat, start_positions[b], window, theta, b)
        scores = (qr.float() @ kr.float().transpose(-1, -2)) / math.sqrt(q.shape[-1])
        out.append(torch.logsumexp(scores.masked_fill(~mask, float("-inf")), dim=-1))
    return torch.cat(out, dim=0)


def prefill_value_grad(
    q: torch.Tensor,
    key_hat: torch.Tensor,
    value_hat: torch.Tensor,
    d_out: torch.Tensor,
    start_positions: Sequence[int],
    *,
    window: int = 4096,
    theta: float = 10000.0,
) -> torch.Tensor:
    """dL/dV̂ of :func:`prefill_attention` for the output gradient ``d_out``
    ([B,QH,T,D]): autograd through ``repeat_kv`` and SDPA in fp32, the value
    leg of what the reference's ``loss.backward()`` forms through its
    closed-loop attention (train_full_model_closed_loop_vq.py:277-304).
    Returns fp32 [B,KVH,T,D]."""

    grads = []
    for b in range(q.shape[0]):
        qr, kr, mask = _rotated_chunk(q, key_hat, start_positions[b], window, theta, b)
        v = value_hat[b : b + 1].float().requires_grad_(True)
        vr = v.repeat_interleave(q.shape[1] // key_hat.shape[1], dim=1)
        out = F.scaled_dot_product_attention(qr.float(), kr.float(), vr, attn_mask=mask, dropout_p=0.0)
        out.backward(d_out[b : b + 1].float())
        grads.append(v.grad)
    return torch.cat(grads, dim=0)


def prefill_qk_grad(
    q: torch.Tensor,
    key_hat: torch.Tensor,
    value_hat: torch.Tensor,
    d_out: torch.Tensor,
    start_positions: Sequence[int],
    *,
    window: int = 4096,
    theta: float = 10000.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """dL/dq and dL/dK̂ (pre-RoPE) of :func:`prefill_attention` for the output
    gradient ``d_out``: autograd in fp32 through the rotary (the model's fp16
    cos/sin), ``repeat_kv`` and SDPA, the query and key legs of the
    reference's ``loss.backward()`` through its closed-loop attention
    (train_full_model_closed_loop_vq.py:277-304).  Returns fp32
    [B,QH,T,D] and [B,KVH,T,D]."""

    head_dim = int(q.shape[-1])
    groups = q.shape[1] // key_hat.shape[1]
    mask = sliding_causal_mask(int(q.shape[2]), window)
    dqs, dks = [], []
    for b in range(q.shape[0]):
        pos = torch.arange(q.shape[2]) + int(start_positions[b])
        c, s = rotary_cos_sin(pos, head_dim, theta)
        qf = q[b : b + 1].float().requires_grad_(True)
        kf = key_hat[b : b + 1].float().requires_grad_(True)
        qr = apply_rotary(qf, c.float()[None, None], s.float()[None, None])
        kr = apply_rotary(kf, c.float()[None, None], s.float()[None, None]).repeat_interleave(groups, dim=1)
        vr = value_hat[b : b + 1].float().repeat_interleave(groups, dim=1)
        out = F.scaled_dot_product_attention(qr, kr, vr, attn_mask=mask, dropout_p=0.0)
        out.backward(d_out[b : b + 1].float())
        dqs.append(qf.grad)
        dks.append(kf.grad)
    return torch.cat(dqs, dim=0), torch.cat(dks, dim=0)


def closed_loop_attention_layer(
    hidden: torch.Tensor,
    weights: dict,
    key_tables: torch.Tensor,
    value_tables: torch.Tensor,
    *,
    depth: int,
    key_whitener: torch.Tensor | None = None,
    window: int = 4096,
    theta: float = 10000.0,
    head_dim: int = 128,
    key_grad: bool = True,
    quantize: bool = True,
    forced_codes: tuple | None = None,
):
    """Forward of one layer of install_closed_loop_attention
    (train_full_model_closed_loop_vq.py:219-337) under autograd: fp16
    projections of ``hidden`` (fp32 accumulate, one rounding), the codec's
    greedy residual VQ on raw K and V (``key_tables`` frozen; full-vector
    ``[KVH,S,K,D]`` or grouped ``[KVH,G,S,K,d]`` tables), RoPE, repeat_kv,
    masked SDPA rounded to fp16, and o_proj in fp32.  ``value_tables`` may
    require grad; with ``key_grad`` the quantized key keeps its
    straight-through edge to ``hidden``.  Returns (projected fp32 [B,T,hidden],
    key search, value search), each search the list [codes, best distance,
    second-best distance] per stage.  ``forced_codes`` (key codes, value
    codes) makes the chains follow another implementation's choices (see
    :func:`hard_residual_vq_exits`).  ``quantize=False`` attends over the raw
    K/V (the unadapted layer; searches None)."""

    batch, tokens, _ = map(int, hidden.shape)
    h32 = hidden.float()

    def proj(w):
        return (h32 @ w.float().T).half()

    qh = weights["q"].shape[0] // head_dim
    kvh = weights["k"].shape[0] // head_dim
    query = proj(weights["q"]).view(batch, tokens, qh, head_dim).transpose(1, 2)
    raw_key = proj(weights["k"]).view(batch, tokens, kvh, head_dim).transpose(1, 2)
    raw_value = proj(weights["v"]).view(batch, tokens, kvh, head_dim).transpose(1, 2)
    forced_k, forced_v = (None, None) if forced_codes is None else forced_codes
    if not quantize:
        k_exits, k_codes, v_exits, v_codes = {depth: raw_key}, None, {depth: raw_value}, None
    elif key_tables.ndim == 5:
        if key_whitener is not None:
            raise ValueError("the oracle's grouped tables take no whitener")
        k_exits, *k_codes = grouped_residual_vq(raw_key, key_tables.detach(), prefixes=(depth,),
                                                return_margins=True, forced_codes=forced_k)
        v_exits, *v_codes = grouped_residual_vq(raw_value, value_tables, prefixes=(depth,), return_margins=True,
                                                forced_codes=forced_v)
    else:
        k_exits, *k_codes = hard_residual_vq_exits(raw_key, key_tables.detach(), prefixes=(depth,),
                                                   assignment_whiteners=key_whitener, return_margins=True,
                                                   forced_codes=forced_k)
        v_exits, *v_codes = hard_residual_vq_exits(raw_value, value_tables, prefixes=(depth,), return_margins=True,
                                                   forced_codes=forced_v)
    khat, vhat = (k_exits[depth] if key_grad else k_exits[depth].detach()), v_exits[depth]
    outs = []
    for b in range(batch):
        pos = torch.arange(tokens)
        c, s = rotary_cos_sin(pos, head_dim, theta)
        qr = apply_rotary(query[b : b + 1].float(), c.float()[None, None], s.float()[None, None])
        kr = apply_rotary(khat[b : b + 1].float(), c.float()[None, None], s.float()[None, None])
        kr = kr.repeat_interleave(qh // kvh, dim=1)
        mask = sliding_causal_mask(tokens, window)
        vr = vhat[b : b + 1].repeat_interleave(qh // kvh, dim=1)
        att = F.scaled_dot_product_attention(qr, kr, vr.float(), attn_mask=mask, dropout_p=0.0)
        outs.append(att.to(torch.float16))
    out = torch.cat(outs, dim=0).transpose(1, 2).reshape(batch, tokens, qh * head_dim)
    return out.float() @ weights["o"].float().T, k_codes, v_codes


def closed_loop_attention_value_step(
    hidden: torch.Tensor,
    weights: dict,
    key_tables: torch.Tensor,
    value_tables: torch.Tensor,
    d_projected: torch.Tensor,
    *,
    depth: int,
    key_whitener: torch.Tensor | None = None,
    window: int = 4096,
    theta: float = 10000.0,
    head_dim: int = 128,
    hidden_grad: bool = False,
):
    """One layer of install_closed_loop_attention
    (train_full_model_closed_loop_vq.py:219-337) followed by backward of a
    given upstream gradient, as the V-only step runs it
    (train_mistral_v_only.py:142-150).  Returns (projected fp16
    [B,T,hidden], dL/d value tables fp32 [KVH,S,K,D]), and with
    ``hidden_grad`` also dL/d hidden (through the codec's straight-through
    edges to raw K and V and the attention's query and key legs)."""

    h32 = hidden.float().requires_grad_(hidden_grad)
    vt = value_tables.detach().clone().requires_grad_(True)
    projected, _kc, _vc = closed_loop_attention_layer(
        h32, weights, key_tables, vt, depth=depth, key_whitener=key_whitener, window=window, theta=theta,
        head_dim=head_dim, key_grad=hidden_grad)
    projected.backward(d_projected.float())
    if hidden_grad:
        return projected.detach().half(), vt.grad, h32.grad
    return projected.detach().half(), vt.grad


def rms_norm(hidden: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Mistral's RMSNorm (transformers 4.45.1 MistralRMSNorm, third-party;
    restated): fp32 x * rsqrt(mean(x^2) + eps), cast to fp16, times the fp16
    weight (one fp16 rounding)."""

    x = hidden.float()
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return (weight.float() * x.half().float()).half()


def causal_loss(logits: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """Mean next-token cross-entropy (train_full_model_closed_loop_vq.py:359-364)."""

    return F.cross_entropy(logits[:, :-1].float().reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1),
                           reduction="mean")


def stack_logits(
    tokens: torch.Tensor,
    stack: dict,
    key_tables: Sequence[torch.Tensor] | None,
    value_tables: Sequence[torch.Tensor] | None,
    *,
    depth: int = 1,
    window: int = 4096,
    theta: float = 10000.0,
    eps: float = 1e-5,
    head_dim: int = 128,
    quantize: bool = True,
    forced_codes: Sequence[tuple] | None = None,
):
    """Logits fp16 [B,T,V] of a Mistral-shaped decoder stack under autograd,
    every layer's attention through :func:`closed_loop_attention_layer`.

    ``stack``: ``embed [V,hidden]``, ``final_norm [hidden]``, ``lm_head
    [V,hidden]`` and ``layers``, each a dict of ``input_norm``,
    ``post_attention_norm``, attention ``q k v o`` and MLP ``gate up down``
    (fp16, ``[out,in]``).  Each decoder layer is Mistral's pre-norm block
    (transformers 4.45.1 MistralDecoderLayer, third-party; restated):
    h += o_proj(attention(norm(h))); h += down(silu(gate(norm(h))) * up(norm(h))),
    every fp16 op rounded once.  ``quantize=False`` runs the unadapted model
    (tables unused).  ``forced_codes``: per layer, (key codes, value codes)
    for :func:`closed_loop_attention_layer`.  Returns the logits and each
    layer's (key search, value search)."""

    h = stack["embed"][tokens]
    codes = []
    for layer, w in enumerate(stack["layers"]):
        x = rms_norm(h, w["input_norm"], eps)
        projected, kc, vc = closed_loop_attention_layer(
            x, w, key_tables[layer] if quantize else None, value_tables[layer] if quantize else None,
            depth=depth, window=window, theta=theta, head_dim=head_dim, quantize=quantize,
            forced_codes=None if forced_codes is None else forced_codes[layer])
        codes.append((kc, vc))
        h = (h.float() + projected.half().float()).half()
        x = rms_norm(h, w["post_attention_norm"], eps).float()
        gate = (x @ w["gate"].float().T).half()
        up = (x @ w["up"].float().T).half()
        act = (F.silu(gate.float()).half().float() * up.float()).half()
        h = (h.float() + (act.float() @ w["down"].float().T).half().float()).half()
    h = rms_norm(h, stack["final_norm"], eps)
    return (h.float() @ stack["lm_head"].float().T).half(), codes


def v_only_stack_step(
    tokens: torch.Tensor,
    stack: dict,
    key_tables: Sequence[torch.Tensor],
    value_tables: Sequence[torch.Tensor],
    *,
    depth: int,
    lr: float = 0.001,
    maximum_norm: float = 1.0,
    window: int = 4096,
    theta: float = 10000.0,
    eps: float = 1e-5,
    head_dim: int = 128,
    forced_codes: Sequence[tuple] | None = None,
) -> dict:
    """One V-only calibration step over a Mistral-shaped decoder stack, in the
    order of train_mistral_v_only.py:143-153: :func:`stack_logits` with every
    layer's attention routed through the codec (install_closed_loop_attention),
    the causal loss, backward, the per_layer_kv clip at ``maximum_norm`` and
    SGD at ``lr``.  Returns the loss, the value-table gradients before
    clipping, the clip record, the updated tables and each layer's (key
    search, value search).  ``forced_codes``: as in :func:`stack_logits`."""

    kts = [t.detach().float().clone() for t in key_tables]
    vts = [torch.nn.Parameter(t.detach().float().clone()) for t in value_tables]
    logits, codes = stack_logits(tokens, stack, kts, vts, depth=depth, window=window, theta=theta, eps=eps,
                                 head_dim=head_dim, forced_codes=forced_codes)
    loss = causal_loss(logits, tokens)
    loss.backward()
    grads = [p.grad.detach().clone() for p in vts]
    keys = [torch.nn.Parameter(t, requires_grad=False) for t in kts]
    clip = clip_codebook_gradients(keys, vts, maximum_norm=maximum_norm, mode="per_layer_kv")
    torch.optim.SGD(vts, lr=lr).step()
    return {"loss": float(loss.detach()), "grads": grads, "clip": clip,
            "value_tables": [p.detach() for p in vts], "codes": codes}


def attention_fp64(q_rot: torch.Tensor, k_rot: torch.Tensor, v: torch.Tensor, mask: torch.Tensor | None = None) -> torch.Tensor:
    """Textbook softmax(q k^T / sqrt(D)) v in fp64 (pin for the SDPA leg)."""

    q64, k64, v64 = q_rot.double(), k_rot.double(), v.double()
    scores = q64 @ k64.transpose(-1, -2) / math.sqrt(q64.shape[-1])
    if mask is not None:
        scores = scores.masked_fill(~mask, float("-inf"))
    return torch.softmax(scores, dim=-1) @ v64


# ---------------------------------------------------------------------------
# Seeded synthetic inputs (fixed generator draw order)


def synthetic_states(generator: torch.Generator, batch: int, heads: int, tokens: int, dim: int = 128,
                     outliers: int = 4, outlier_scale: float = 8.0) -> torch.Tensor:
    """N(0,1) states with ``outliers`` random channels per head scaled, as fp16."""

    x = torch.randn(batch, heads, tokens, dim, generator=generator)
    for h in range(heads):
        channels = torch.randperm(dim, generator=generator)[:outliers]
        x[:, h, :, channels] *= outlier_scale
    return x.half()


def synthetic_tables(generator: torch.Generator, shape, stage_sigmas: Sequence[float], stage_axis: int) -> torch.Tensor:
    """fp16-valued fp32 codebooks; stage s drawn N(0, sigma_s^2)."""

    t = torch.randn(*shape, generator=generator)
    for s, sigma in enumerate(stage_sigmas):
        index = [slice(None)] * len(shape)
        index[stage_axis] = s
        t[tuple(index)] *= sigma
    return t.half().float()
