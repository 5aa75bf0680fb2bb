#!/usr/bin/env python3
"""Benchmark of the jointkv hard residual-quantization hot path on one MI355X.

Headline line: GSRQ-2 encode of a Mistral-7B-shaped
cache, 32 layers x {K,V} x [1,8,8192,128] fp16 with 4 outlier channels per
head, 16 groups x 8 dims x 2 residual stages x 256 fp16 codewords per
(head, group) (stage 1 N(0,1), stage 2 N(0,0.25)), codes + fp16
reconstruction written.  One step = the 64 encodes of the whole cache in one
call and one launch (`rvq_encode_many`); the same 64 encodes as 32 launches
(a layer's K and V per launch, as the codec forward issues them during a
forward pass) and as 64 launches are reported beside it.

Extra measurements in the same JSON line:
  decode   config 4: fused packed-code GQA decode (32q/8kv, B16, 4096 window,
           G2 codes), one new token per step over 32 layers (encode + append +
           attention per layer), us/step
  prefill  config 4: 2048-token causal prefill chunk (B16, 32q/8kv), us per
           layer and MFMA fraction
  vstack   config 5 as the reference runs it: the V-only step over a
           synthetic 32-layer Mistral-7B-shaped decoder (batch 4, 2048
           tokens), forward + backward through the stack, per_layer_kv clip,
           SGD; steps/s
  vstep    config 5: V-only STE calibration step over 32 layers at
           [4,8,2048,128] (encode fwd, scatter bwd, global clip, SGD), steps/s,
           with the layers' encodes and scatters batched (and per layer)
  cq2      config 3: reference cq2 grouped-CQ encode ([8,32,256,4]) of
           32 layers x {K,V} x [4,8,2048,128] in one call (and per layer),
           tokens/s
  roofline of the encode kernel (MFMA, algorithmic flops) and cpu_baseline
  (the oracle's eager-PyTorch restatement of the reference on a bounded
  sample, timed on this host).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tac-vq-kv-cache_amd"))
sys.path.insert(0, str(ROOT))

MFMA_FP16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBS = 8000.0

LAYERS = 32
HEADS = 8
HEAD_DIM = 128
GROUPS = 16
GROUP_DIM = 8
STAGES = 2
CLUSTERS = 256
FLOP_PER_VEC_G2 = STAGES * GROUPS * CLUSTERS * GROUP_DIM * 2  # 131072


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_states(gen, batch, heads, tokens, device):
    import torch

    x = torch.randn(batch, heads, tokens, HEAD_DIM, generator=gen, device=device)
    for h in range(heads):
        ch = torch.randperm(HEAD_DIM, generator=gen, device=device)[:4]
        x[:, h, :, ch] *= 8.0
    return x.half()


def make_tables(gen, shape, sigmas, stage_axis, device):
    import torch

    t = torch.randn(*shape, generator=gen, device=device)
    for s, sg in enumerate(sigmas):
        idx = [slice(None)] * len(shape)
        idx[stage_axis] = s
        t[tuple(idx)] *= sg
    return t.half().float().contiguous()


def timed(fn, steps, warmup):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # a spin kernel ahead of the start event keeps the stream busy while the
    # host enqueues the first step, so the events time the steps themselves
    # (back to back) and not the host's enqueue of the first one
    torch.cuda._sleep(20_000_000)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms per step


def per_launch_ms(launches, repeats: int = 3) -> float:
    """Average time of one call in `launches`, from two HIP events on the
    launching stream around all of them.  A spin kernel queued first keeps the
    stream busy while the host enqueues, so the calls run back to back and the
    events time the kernels rather than host launch gaps.  Median of
    `repeats` passes."""

    import torch

    passes = []
    for _ in range(repeats):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        torch.cuda._sleep(100_000_000)
        a.record()
        for fn in launches:
            fn()
        b.record()
        torch.cuda.synchronize()
        passes.append(a.elapsed_time(b) / len(launches))
    return sorted(passes)[len(passes) // 2]


def measured_traffic(kernel_profile: Path) -> int | None:
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE + WRITE_SIZE
    (scaled by a copy-kernel calibration), read from the committed profile
    summary; None when the summary is absent."""

    if not kernel_profile.is_file():
        return None
    for line in kernel_profile.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def copy_calibration() -> None:
    """A plain 256 MiB device copy, four times: profiled with FETCH_SIZE and
    WRITE_SIZE it gives the counters' scale (reads 256 MiB, writes 256 MiB per
    dispatch)."""

    import torch

    x = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    x.fill_(1.0)
    for _ in range(4):
        y.copy_(x)
    torch.cuda.synchronize()
    log("copy calibration: 4 x (256 MiB read + 256 MiB written)")


def encode_workload(args, device):
    import torch
    from jointkv_amd import _ops

    gen = torch.Generator(device=device).manual_seed(8601)
    layers = []
    for _layer in range(LAYERS):
        kv = []
        for _kind in range(2):
            states = make_states(gen, 1, HEADS, args.tokens, device)
            tables = make_tables(gen, (HEADS * GROUPS, STAGES, CLUSTERS, GROUP_DIM), (1.0, 0.5), 1, device)
            kv.append((states, tables))
        layers.append(kv)
    log(f"encode inputs ready: {LAYERS} layers x {{K,V}} of {tuple(layers[0][0][0].shape)}")

    flat_states = [states for kv in layers for states, _ in kv]
    flat_tables = [tables for kv in layers for _, tables in kv]

    # the whole cache in one call: every layer's K and V in one launch
    def step():
        _ops.rvq_encode_many(flat_states, flat_tables, groups=GROUPS, group_dim=GROUP_DIM, exits=(STAGES,))

    # the codec forward of a layer encodes its K and V (uniform_depth_tac.py:
    # 69-101): one launch per layer, both tensors' workgroups in one grid
    def step_per_layer():
        for (ks, kt), (vs, vt) in layers:
            _ops.rvq_encode_kv(ks, vs, kt, vt, groups=GROUPS, group_dim=GROUP_DIM, exits=(STAGES,))

    def step_separate():
        for kv in layers:
            for states, tables in kv:
                _ops.rvq_encode(states, tables, groups=GROUPS, group_dim=GROUP_DIM, exits=(STAGES,))

    ms = timed(step, args.steps, args.warmup)
    ms_per_layer = timed(step_per_layer, args.steps, args.warmup)
    ms_separate = timed(step_separate, args.steps, args.warmup)
    # the timed region's HIP events over its back-to-back launches: the host
    # enqueues a step in well under its ~2 ms of GPU time, so the queue never
    # drains and the average is the kernel's own duration
    vecs_per_launch = 2 * LAYERS * HEADS * args.tokens  # every layer's K and V
    flops_per_launch = vecs_per_launch * FLOP_PER_VEC_G2
    bytes_per_launch = LAYERS * (2 * HEADS * args.tokens * (HEAD_DIM * 2 + GROUPS * STAGES + HEAD_DIM * 2)
                                 + 2 * HEADS * GROUPS * STAGES * CLUSTERS * GROUP_DIM * 4)
    return {
        "ms_per_step": ms,
        "tokens_per_s": args.tokens / (ms / 1e3),
        "vecs_per_s": 2 * LAYERS * HEADS * args.tokens / (ms / 1e3),
        "avg_launch_ms": ms,
        "flops_per_launch": flops_per_launch,
        "bytes_per_launch": bytes_per_launch,
        "launches_per_step": 1,
        "per_layer_launches": {"ms_per_step": ms_per_layer, "tokens_per_s": args.tokens / (ms_per_layer / 1e3),
                               "us_per_launch": ms_per_layer / len(layers) * 1e3},
        "separate_launches": {"ms_per_step": ms_separate, "tokens_per_s": args.tokens / (ms_separate / 1e3),
                              "us_per_launch": ms_separate / (2 * len(layers)) * 1e3},
    }


def cq2_workload(args, device):
    import torch
    from jointkv_amd import _ops

    gen = torch.Generator(device=device).manual_seed(8601)
    tensors = []
    for _ in range(LAYERS * 2):
        states = make_states(gen, 4, HEADS, 2048, device)
        books = make_tables(gen, (HEADS * 32, 1, CLUSTERS, 4), (1.0,), 1, device)
        tensors.append((states, books))

    # the whole cache in one call (one launch)
    def step():
        _ops.rvq_encode_many([t[0] for t in tensors], [t[1] for t in tensors], groups=32, group_dim=4, exits=(1,))

    # a layer's K and V per launch, as the codec forward issues them
    def step_per_layer():
        for (ks, kb), (vs, vb) in zip(tensors[0::2], tensors[1::2]):
            _ops.rvq_encode_kv(ks, vs, kb, vb, groups=32, group_dim=4, exits=(1,))

    ms = timed(step, max(1, args.steps // 2), 1)
    ms_per_layer = timed(step_per_layer, max(1, args.steps // 2), 1)
    return {"ms_per_step": ms, "tokens_per_s": 4 * 2048 / (ms / 1e3),
            "per_layer_launches": {"ms_per_step": ms_per_layer, "tokens_per_s": 4 * 2048 / (ms_per_layer / 1e3)}}


def full_vector_workload(args, device):
    """Config 3 read literally: two full-vector (d = 128) residual stages per
    (layer, K/V), 32 layers x {K,V} x [4,8,2048,128], tables [8,2,256,128]."""
    import torch
    from jointkv_amd import _ops

    gen = torch.Generator(device=device).manual_seed(8601)
    tensors = []
    for _ in range(LAYERS * 2):
        states = make_states(gen, 4, HEADS, 2048, device)
        tables = make_tables(gen, (HEADS, 2, CLUSTERS, HEAD_DIM), (1.0, 0.5), 1, device)
        tensors.append((states, tables))

    # the whole cache in one call: every tensor's tables in one launch, every
    # tensor's search in another
    def step():
        _ops.rvq_encode_many([t[0] for t in tensors], [t[1] for t in tensors], groups=1, group_dim=HEAD_DIM,
                             exits=(2,))

    # one call per tensor, as the codec forward issues them
    def step_per_tensor():
        for states, tables in tensors:
            _ops.rvq_encode(states, tables, groups=1, group_dim=HEAD_DIM, exits=(2,))

    ms = timed(step, max(1, args.steps // 2), 1)
    ms_per_tensor = timed(step_per_tensor, max(1, args.steps // 2), 1)
    vecs = 4 * HEADS * 2048
    flops = vecs * 2 * CLUSTERS * HEAD_DIM * 2  # two stages, 256 codewords, 128 dims, multiply-add
    launch_us = ms * 1e3 / len(tensors)
    return {
        "ms_per_step": ms,
        "tokens_per_s": 4 * 2048 / (ms / 1e3),
        "us_per_encode": launch_us,
        "tflops": flops / (launch_us * 1e-6) / 1e12,
        "mfma_frac": flops / (launch_us * 1e-6) / 1e12 / MFMA_FP16_PEAK_TFLOPS,
        "per_tensor_calls": {"ms_per_step": ms_per_tensor, "us_per_encode": ms_per_tensor * 1e3 / len(tensors)},
    }


def decode_workload(args, device):
    import torch
    import jointkv_amd as jkv
    from jointkv_amd import _ops

    batch, qh, kvh, window = 16, 32, 8, 4096
    gen = torch.Generator(device=device).manual_seed(8601)
    caches, tabs = [], []
    for _ in range(LAYERS):
        kt = make_tables(gen, (kvh * GROUPS, STAGES, CLUSTERS, GROUP_DIM), (1.0, 0.5), 1, device)
        vt = make_tables(gen, (kvh * GROUPS, STAGES, CLUSTERS, GROUP_DIM), (1.0, 0.5), 1, device)
        cache = jkv.PackedCodeCache(batch, kvh, GROUPS, STAGES, capacity=window, device=device)
        codes = torch.randint(0, 256, (batch, kvh, window - 1, GROUPS, STAGES), generator=gen, device=device,
                              dtype=torch.uint8)
        cache.append(codes, codes.roll(1, dims=2))
        caches.append(cache)
        tabs.append((kt, vt, _ops.f32_to_f16(kt), _ops.f32_to_f16(vt)))
    q = torch.randn(batch, qh, HEAD_DIM, generator=gen, device=device).half()
    knew = make_states(gen, batch, kvh, 1, device)
    vnew = make_states(gen, batch, kvh, 1, device)
    lengths = torch.full((batch,), window, dtype=torch.int32, device=device)
    slot = (window - 1) % window

    knew3, vnew3 = knew[:, :, 0], vnew[:, :, 0]

    def step():
        # one launch per layer encodes the new token's K and V into its cache
        # slot and attends over the window with it
        for cache, (_kt, _vt, kt16, vt16) in zip(caches, tabs):
            _ops.decode_attention(q, cache.key, cache.value, kt16, vt16, lengths, window=window,
                                  rope_theta=10000.0, max_length=window, key_new=knew3, value_new=vnew3)

    def step_unfused():
        # the same step with the encode as its own launch
        for cache, (kt, vt, kt16, vt16) in zip(caches, tabs):
            _ops.rvq_encode_kv(knew, vnew, kt, vt, groups=GROUPS, group_dim=GROUP_DIM, exits=(),
                               key_codes_out=cache.key[:, :, slot : slot + 1],
                               value_codes_out=cache.value[:, :, slot : slot + 1])
            _ops.decode_attention(q, cache.key, cache.value, kt16, vt16, lengths, window=window,
                                  rope_theta=10000.0, max_length=window)

    ms = timed(step, args.steps, args.warmup)
    unfused_ms = timed(step_unfused, args.steps, 1)
    # attention kernels alone
    def attn_only():
        for cache, (_kt, _vt, kt16, vt16) in zip(caches, tabs):
            _ops.decode_attention(q, cache.key, cache.value, kt16, vt16, lengths, window=window,
                                  rope_theta=10000.0, max_length=window)

    attn_ms = timed(attn_only, args.steps, 1)
    attn_layer_ms = per_launch_ms(
        [lambda c=c, t=t: _ops.decode_attention(q, c.key, c.value, t[2], t[3], lengths, window=window,
                                                rope_theta=10000.0, max_length=window)
         for c, t in zip(caches, tabs)])
    bytes_per_layer = 2 * batch * kvh * window * GROUPS * STAGES + 2 * kvh * GROUPS * STAGES * CLUSTERS * GROUP_DIM * 2 + 2 * batch * qh * HEAD_DIM * 2
    return {
        "us_per_step": ms * 1e3,
        "us_per_step_encode_separate": unfused_ms * 1e3,
        "attention_us_per_step": attn_ms * 1e3,
        "attention_kernels_us_per_layer": attn_layer_ms * 1e3,
        "hbm_bytes_per_step": bytes_per_layer * LAYERS,
        "hbm_frac": bytes_per_layer * LAYERS / (attn_ms / 1e3) / (HBM_PEAK_GBS * 1e9),
    }


def full_decode_workload(args, device):
    """Packed-code decode for the reference's full-vector codecs (one 128-dim
    group, R16 / R32: 16 or 32 stages of 256 fp16 codewords per kv head,
    train_mistral_v_only.py:58-62) at config 4's shape (B16, 32/8 heads,
    4096-token window): us per layer, and the decoded-window path
    (evaluate_mistral_longbench.py:44-70) over the same shape."""

    import torch
    from jointkv_amd import _ops

    batch, qh, kvh, window = 16, 32, 8, 4096
    gen = torch.Generator(device=device).manual_seed(8611)
    q = torch.randn(batch, qh, HEAD_DIM, generator=gen, device=device).half()
    lengths = torch.full((batch,), window, dtype=torch.int32, device=device)
    out = {}
    for stages in (16, 32):
        sig = torch.tensor([0.8 ** s for s in range(stages)], device=device)
        kt = (torch.randn(kvh, stages, CLUSTERS, HEAD_DIM, generator=gen, device=device) * sig[None, :, None, None]).half()
        vt = (torch.randn(kvh, stages, CLUSTERS, HEAD_DIM, generator=gen, device=device) * sig[None, :, None, None]).half()
        kc = torch.randint(0, 256, (batch, kvh, window, 1, stages), generator=gen, device=device, dtype=torch.uint8)
        vc = torch.randint(0, 256, (batch, kvh, window, 1, stages), generator=gen, device=device, dtype=torch.uint8)
        f = lambda: _ops.decode_attention(q, kc, vc, kt, vt, lengths, window=window, rope_theta=10000.0,
                                          max_length=window)
        out[f"r{stages}_packed_us_per_layer"] = per_launch_ms([f] * 20) * 1e3
        # codeword bytes gathered per layer (K and V), the path's L2 traffic
        out[f"r{stages}_gathered_bytes_per_layer"] = 2 * batch * kvh * window * stages * CLUSTERS
    kw = torch.randn(batch, kvh, window, HEAD_DIM, generator=gen, device=device).half()
    vw = torch.randn(batch, kvh, window, HEAD_DIM, generator=gen, device=device).half()
    f = lambda: _ops.decode_attention_window(q, kw, vw, lengths, window=window, rope_theta=10000.0,
                                             max_length=window)
    out["decoded_window_us_per_layer"] = per_launch_ms([f] * 20) * 1e3
    return out


def prefill_workload(args, device):
    """Config 4 prefill chunk: 2048 tokens, B16, 32/8 heads, causal with the
    4096 sliding window, fp16 K/V as the codec reconstructs them; 32 layers
    per step over 4 distinct layer inputs (1.5 GiB, beyond the caches)."""

    import torch
    from jointkv_amd import _ops

    batch, qh, kvh, tokens = 16, 32, 8, 2048
    gen = torch.Generator(device=device).manual_seed(8601)
    inputs = []
    for _ in range(4):
        q = torch.randn(batch, qh, tokens, HEAD_DIM, generator=gen, device=device).half()
        k = torch.randn(batch, kvh, tokens, HEAD_DIM, generator=gen, device=device).half()
        v = torch.randn(batch, kvh, tokens, HEAD_DIM, generator=gen, device=device).half()
        inputs.append((q, k, v))
    starts = torch.zeros(batch, dtype=torch.int32, device=device)

    def layer(i):
        q, k, v = inputs[i % len(inputs)]
        return _ops.prefill_attention(q, k, v, starts, window=4096, rope_theta=10000.0, max_position=tokens - 1)

    ms = timed(lambda: [layer(i) for i in range(LAYERS)], max(1, args.steps // 2), 1)
    layer_ms = per_launch_ms([lambda i=i: layer(i) for i in range(LAYERS)])
    flops = 4.0 * batch * qh * HEAD_DIM * tokens * (tokens + 1) / 2  # causal QK^T + PV
    return {
        "ms_per_step": ms,
        "us_per_layer": layer_ms * 1e3,
        "tflops": flops / (layer_ms / 1e3) / 1e12,
        "mfma_frac": flops / (layer_ms / 1e3) / 1e12 / MFMA_FP16_PEAK_TFLOPS,
    }


def vstep_workload(args, device):
    import torch
    from jointkv_amd import _ops
    import jointkv_amd as jkv

    gen = torch.Generator(device=device).manual_seed(8601)
    values = [make_states(gen, 4, HEADS, 2048, device) for _ in range(LAYERS)]
    masters = [torch.nn.Parameter(make_tables(gen, (HEADS * GROUPS, STAGES, CLUSTERS, GROUP_DIM), (1.0, 0.5), 1, device))
               for _ in range(LAYERS)]
    upstream = [(torch.randn(4, HEADS, 2048, HEAD_DIM, generator=gen, device=device) * 1e-3 ** 0.5).half()
                for _ in range(LAYERS)]

    class Codec:
        key_tables = []
        value_tables = masters

    def step():
        for p in masters:
            p.grad = None
        # the 32 layers' V states are given, so their encodes share one launch
        encoded = _ops.rvq_encode_many(values, [p.detach() for p in masters], groups=GROUPS,
                                       group_dim=GROUP_DIM, exits=(STAGES,))
        # and their table gradients one scatter launch, stored into fresh
        # tables (no zero fill)
        grads = _ops.rvq_scatter_grad_many([[g] for g in upstream], [STAGES], [c for _, c in encoded],
                                           group_dim=GROUP_DIM, table_shape=masters[0].shape)
        for p, grad in zip(masters, grads):
            p.grad = grad
        jkv.clip_codebook_gradients(Codec, maximum_norm=1.0, mode="global")
        jkv.sgd_step(masters, lr=0.001)

    # the same step with a launch per layer for each encode and each scatter
    # (and a zero-filled gradient per table), as a codec forward and its
    # autograd backward issue them inside a model
    def step_per_layer():
        for p in masters:
            p.grad = None
        for x, p, g in zip(values, masters, upstream):
            _recon, codes = _ops.rvq_encode(x, p.detach(), groups=GROUPS, group_dim=GROUP_DIM, exits=(STAGES,))
            grad = torch.zeros_like(p)
            _ops.rvq_scatter_grad([g], [STAGES], codes, grad, group_dim=GROUP_DIM)
            p.grad = grad
        jkv.clip_codebook_gradients(Codec, maximum_norm=1.0, mode="global")
        jkv.sgd_step(masters, lr=0.001)

    ms = timed(step, max(1, args.steps // 2), 1)
    ms_per_layer = timed(step_per_layer, max(1, args.steps // 2), 1)
    return {"ms_per_step": ms, "steps_per_s": 1e3 / ms,
            "per_layer_launches": {"ms_per_step": ms_per_layer, "steps_per_s": 1e3 / ms_per_layer}}


def adapter_workload(args, device):
    """One decoder layer of the closed-loop attention adapter at config 5's
    shape (batch 4, 2048 tokens, 8 kv heads; Mistral hidden 4096, 32 query
    heads): projections, GSRQ-2 encode of K and V, prefill attention with its
    row normaliser, o_proj, then backward of a synthetic upstream gradient
    into the value tables (o_proj backward GEMM, HIP value gradient, HIP
    scatter-add).  Random weights; the value-gradient kernel is also timed
    alone."""

    import torch
    import jointkv_amd as jkv
    from jointkv_amd import _ops
    from jointkv_amd.closed_loop_attention import AttentionWeights, closed_loop_attention

    batch, tokens, hidden_size, qh = 4, 2048, 4096, 32
    gen = torch.Generator(device=device).manual_seed(8601)
    hidden = (torch.randn(batch, tokens, hidden_size, generator=gen, device=device) * 0.5).half()
    w = [(torch.randn(rows, hidden_size, generator=gen, device=device) / hidden_size ** 0.5).half()
         for rows in (hidden_size, HEADS * HEAD_DIM, HEADS * HEAD_DIM, hidden_size)]
    weights = AttentionWeights(*w)
    shape = (HEADS, GROUPS, STAGES, CLUSTERS, GROUP_DIM)
    ktab = make_tables(gen, shape, (1.0, 0.5), 2, device)
    vtab = make_tables(gen, shape, (1.0, 0.5), 2, device)
    codec = jkv.ClosedLoopUniformResidualVQ([ktab], [vtab], [None], depth=STAGES, dynamic_bpa=2.0).to(device)
    upstream = (torch.randn(batch, tokens, hidden_size, generator=gen, device=device) * 1e-3 ** 0.5).half()

    def step():
        codec.value_tables[0].grad = None
        out = closed_loop_attention(hidden, weights, codec, 0)
        out.backward(upstream)

    ms = timed(step, max(1, args.steps // 2), 1)
    # the value-gradient kernel alone
    q = torch.randn(batch, qh, tokens, HEAD_DIM, generator=gen, device=device).half()
    k = torch.randn(batch, HEADS, tokens, HEAD_DIM, generator=gen, device=device).half()
    v = torch.randn(batch, HEADS, tokens, HEAD_DIM, generator=gen, device=device).half()
    d = torch.randn(batch, qh, tokens, HEAD_DIM, generator=gen, device=device).half()
    starts = torch.zeros(batch, dtype=torch.int32, device=device)
    lse = torch.empty(batch, qh, tokens, dtype=torch.float32, device=device)
    _ops.prefill_attention(q, k, v, starts, window=4096, rope_theta=10000.0, max_position=tokens - 1, lse=lse)
    launches = [lambda: _ops.prefill_attention_value_grad(q, k, d, lse, starts, window=4096, rope_theta=10000.0,
                                                          max_position=tokens - 1)] * 8
    dv_ms = per_launch_ms(launches)
    flops = 4.0 * batch * qh * HEAD_DIM * tokens * (tokens + 1) / 2  # causal S recompute + Pᵀ dO
    # the full backward (query, key and value legs), as a lower layer of the
    # trajectory needs it
    out = _ops.prefill_attention(q, k, v, starts, window=4096, rope_theta=10000.0, max_position=tokens - 1,
                                 lse=lse)
    full = [lambda: _ops.prefill_attention_backward(q, k, v, out, d, lse, starts, window=4096, rope_theta=10000.0,
                                                    max_position=tokens - 1)] * 4
    bwd_ms = per_launch_ms(full)
    bwd_flops = 4 * flops  # S recompute, dP, dS K̂ and dSᵀ Q, Pᵀ dO (the key leg recomputes S and dP)
    return {
        "ms_per_layer_step": ms,
        "value_grad_us": dv_ms * 1e3,
        "value_grad_tflops": flops / (dv_ms / 1e3) / 1e12,
        "value_grad_mfma_frac": flops / (dv_ms / 1e3) / 1e12 / MFMA_FP16_PEAK_TFLOPS,
        "full_backward_us": bwd_ms * 1e3,
        "full_backward_tflops_algorithmic": 2.5 * flops / (bwd_ms / 1e3) / 1e12,
    }


def vstack_workload(args, device):
    """The V-only calibration step over a synthetic 32-layer Mistral-7B-shaped
    decoder at config 5's shape (batch 4, 2048 tokens; hidden 4096, 32 query /
    8 kv heads, MLP 14336, vocabulary 32000; random frozen fp16 weights,
    random token ids), every layer's K/V through a GSRQ-2 codec, in the
    order of train_mistral_v_only.py:143-153: forward, causal loss, checks,
    backward (value leg in the first layer, full attention backward above
    it), per_layer_kv clip at 1.0, SGD at lr 0.001."""

    import torch
    import jointkv_amd as jkv
    from jointkv_amd.v_only import ClosedLoopRunContext, DecoderStack, run_loss, v_only_step

    batch, tokens, vocab, inter = 4, 2048, 32000, 14336
    gen = torch.Generator(device=device).manual_seed(8601)
    stack = DecoderStack.synthetic(gen, layers=LAYERS, hidden=HEADS * 4 * HEAD_DIM, kv_heads=HEADS,
                                   intermediate=inter, vocab=vocab)
    shape = (HEADS, GROUPS, STAGES, CLUSTERS, GROUP_DIM)
    ktabs = [make_tables(gen, shape, (1.0, 0.5), 2, device) for _ in range(LAYERS)]
    vtabs = [make_tables(gen, shape, (1.0, 0.5), 2, device) for _ in range(LAYERS)]
    codec = jkv.ClosedLoopUniformResidualVQ(ktabs, vtabs, [None] * LAYERS, depth=STAGES, dynamic_bpa=2.0).to(device)
    context = ClosedLoopRunContext(codec, "uniform")
    ids = torch.randint(0, vocab, (batch, tokens), generator=gen, device=device)
    log(f"stacked V-only step: {LAYERS} layers, hidden {HEADS * 4 * HEAD_DIM}, MLP {inter}, batch {batch} x {tokens}")
    count = [0]

    def step():
        v_only_step(context, lambda: run_loss(stack, context, ids, mode="uniform"), step=count[0])
        count[0] += 1

    ms = timed(step, 2, 1)
    peak = torch.cuda.max_memory_allocated(device)
    del stack, codec, context
    torch.cuda.empty_cache()
    return {"ms_per_step": ms, "steps_per_s": 1e3 / ms, "layers": LAYERS, "batch": batch, "tokens": tokens,
            "hidden": HEADS * 4 * HEAD_DIM, "intermediate": inter, "vocab": vocab, "clip": "per_layer_kv 1.0",
            "peak_hbm_gib": peak / 2 ** 30}


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_seconds(fn, runs: int = 3) -> float:
    fn()  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_baseline(args):
    """The oracle (eager PyTorch restatement of the reference's op sequence)
    timed on this host with every core, median of 3 after a warm-up.

    Headline (config 2): one (layer, K) tensor over a bounded token sample,
    scaled to tokens/s of the full 32-layer x {K,V} workload.  Alongside:
    config 1 at full size (grouped CQ of one layer's K and V,
    cq_tac.py:33-114) and one config-4 decode layer at batch 16 (decode the
    codes, RoPE, repeat_kv, SDPA: evaluate_mistral_longbench.py:112-122),
    scaled x32 layers."""

    import torch
    from oracle import jointkv_oracle as ref

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(8601)
    tokens = args.cpu_tokens
    states = ref.synthetic_states(gen, 1, HEADS, tokens)
    tables = ref.synthetic_tables(gen, (HEADS, GROUPS, STAGES, CLUSTERS, GROUP_DIM), (1.0, 0.5), stage_axis=2)
    with torch.no_grad():
        sec = _median_seconds(lambda: ref.grouped_residual_vq(states, tables, prefixes=(2,)))
    # one (layer, K) tensor of `tokens` tokens took `sec`; a full token needs 64 such
    per_token = sec / tokens * (2 * LAYERS)

    # config 1: cq1 K and V of one layer at full size, token_chunk_size 64
    gen1 = torch.Generator().manual_seed(8601)
    k1 = ref.synthetic_states(gen1, 1, HEADS, 2048)
    v1 = ref.synthetic_states(gen1, 1, HEADS, 2048)
    books = ref.synthetic_tables(gen1, (HEADS, GROUPS, CLUSTERS, GROUP_DIM), (1.0,), stage_axis=0)
    with torch.no_grad():
        sec1 = _median_seconds(lambda: (ref.hard_grouped_cq(k1, books), ref.hard_grouped_cq(v1, books)))

    # config 4: one decode layer, B16, 32 query / 8 kv heads, 4096 cached tokens
    gen4 = torch.Generator().manual_seed(8601)
    b4, window = 16, 4096
    q = torch.randn(b4, 32, 1, HEAD_DIM, generator=gen4).half()
    kc = torch.randint(0, CLUSTERS, (b4, HEADS, window, GROUPS, STAGES), generator=gen4, dtype=torch.uint8)
    vc = torch.randint(0, CLUSTERS, (b4, HEADS, window, GROUPS, STAGES), generator=gen4, dtype=torch.uint8)
    kt = ref.synthetic_tables(gen4, (HEADS * GROUPS, STAGES, CLUSTERS, GROUP_DIM), (1.0, 0.5), stage_axis=1)
    vt = ref.synthetic_tables(gen4, (HEADS * GROUPS, STAGES, CLUSTERS, GROUP_DIM), (1.0, 0.5), stage_axis=1)
    pos = torch.arange(window)

    def decode_layer():
        khat = ref.frozen_decode(kc, kt, STAGES, torch.float16)
        vhat = ref.frozen_decode(vc, vt, STAGES, torch.float16)
        return ref.decode_attention(q, khat, vhat, window - 1, pos)

    with torch.no_grad():
        sec4 = _median_seconds(decode_layer)
    return {
        "value": 1.0 / per_token,
        "unit": "tokens/s",
        "cores": int(torch.get_num_threads()),
        "kind": "port",
        "sample": f"oracle grouped_residual_vq (reference op sequence, token_chunk_size=1024) on one "
                  f"(layer,K) tensor [1,8,{tokens},128], median of 3 after a warm-up, scaled x64 tensors per token",
        "host": {"cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(),
                 "torch_threads": int(torch.get_num_threads()), "torch": torch.__version__},
        "config1_full": {"ms_per_layer_kv": sec1 * 1e3,
                         "sample": "oracle hard_grouped_cq of K and V [1,8,2048,128], codebooks [8,16,256,8], "
                                   "token_chunk_size 64, full size, median of 3"},
        "config4_decode": {"us_per_step": sec4 * LAYERS * 1e6, "ms_per_layer": sec4 * 1e3,
                           "sample": "oracle frozen_decode (K and V, G2 codes [16,8,4096,16,2]) + rotary + "
                                     "repeat_kv + SDPA for q [16,32,1,128], one layer, median of 3, scaled x32"},
    }


def cq1_workload(args, device):
    """Config 1 on the GPU: cq1 (16 groups x 8 dims, 256 codewords) K and V
    of one layer [1,8,2048,128], as the codec forward encodes them."""

    import torch
    from jointkv_amd import _ops

    gen = torch.Generator(device=device).manual_seed(8601)
    k = make_states(gen, 1, HEADS, 2048, device)
    v = make_states(gen, 1, HEADS, 2048, device)
    books = make_tables(gen, (HEADS * GROUPS, 1, CLUSTERS, GROUP_DIM), (1.0,), 1, device)
    vbooks = make_tables(gen, (HEADS * GROUPS, 1, CLUSTERS, GROUP_DIM), (1.0,), 1, device)
    launches = [lambda: _ops.rvq_encode_kv(k, v, books, vbooks, groups=GROUPS, group_dim=GROUP_DIM, exits=(1,))]
    launches[0]()
    us = per_launch_ms(launches * 100) * 1e3
    return {"us_per_layer_kv": us}


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=10)
    parser.add_argument("--warmup", type=int, default=2)
    parser.add_argument("--tokens", type=int, default=8192)
    parser.add_argument("--cpu-tokens", type=int, default=2048)
    parser.add_argument("--skip", default="", help="comma list of extras to skip: decode,rdecode,prefill,vstep,vstack,adapter,cq1,cq2,full,cpu")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run the 256 MiB copy used to scale FETCH_SIZE/WRITE_SIZE")
    args = parser.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the hot path has no multi-GPU leg "
              "(its kv heads shard across GPUs with no exchange between them)", file=sys.stderr)
        return 2
    import torch

    skip = set(filter(None, args.skip.split(",")))
    device = torch.device("cuda:0")
    log("encode workload (config 2)")
    enc = encode_workload(args, device)
    log(f"encode: {enc['ms_per_step']:.3f} ms/step")
    extras = {}
    if "cq1" not in skip:
        log("cq1 workload (config 1)")
        extras["cq1_encode"] = cq1_workload(args, device)
    if "cq2" not in skip:
        log("cq2 workload (config 3)")
        extras["cq2_encode"] = cq2_workload(args, device)
    if "full" not in skip:
        log("full-vector workload (config 3, literal two-stage reading)")
        extras["full_vector_encode"] = full_vector_workload(args, device)
    if "decode" not in skip:
        log("decode workload (config 4)")
        extras["decode"] = decode_workload(args, device)
    if "rdecode" not in skip:
        log("full-vector (R16/R32) packed decode ...")
        extras["full_vector_decode"] = full_decode_workload(args, device)
    if "prefill" not in skip:
        log("prefill workload (config 4 prefill chunk)")
        extras["prefill"] = prefill_workload(args, device)
    if "vstep" not in skip:
        log("V-only step workload (config 5)")
        extras["v_only_step"] = vstep_workload(args, device)
    if "vstack" not in skip:
        log("stacked V-only step (config 5 shape, 32 Mistral-7B-shaped layers) ...")
        extras["v_only_stack_step"] = vstack_workload(args, device)
    if "adapter" not in skip:
        log("closed-loop attention layer step (config 5 shape)")
        extras["closed_loop_attention"] = adapter_workload(args, device)
    cpu = None
    if "cpu" not in skip:
        log("cpu baseline")
        cpu = cpu_baseline(args)
    achieved = enc["flops_per_launch"] / (enc["avg_launch_ms"] / 1e3) / 1e12
    record = {
        "metric": "GSRQ-2 encode tokens/s (32 layers x {K,V} x [1,8,8192,128], G2 16x8x2x256)",
        "value": enc["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": enc["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (fp32 accumulate)",
        "data": "synthetic: seeded N(0,1) states with 4 x8 outlier channels per head; seeded codebooks",
        "config": {
            "workload": "BASELINE config 2: GSRQ-2 grouped residual encode + fp16 reconstruction",
            "layers": LAYERS, "kv_heads": HEADS, "tokens": args.tokens, "batch": 1,
            "groups": GROUPS, "group_dim": GROUP_DIM, "stages": STAGES, "codewords": CLUSTERS,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": achieved,
            "peak": MFMA_FP16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / MFMA_FP16_PEAK_TFLOPS,
            "traffic": measured_traffic(ROOT / "profiles" / "rvq_encode_grouped_g2_config2.md"),
            "kernel": "rvq_encode_grouped<8,2,many> (every layer's K and V in one launch)",
            "avg_launch_us": enc["avg_launch_ms"] * 1e3,
            "algorithmic_flop_per_launch": enc["flops_per_launch"],
            "algorithmic_bytes_per_launch": enc["bytes_per_launch"],
            "hbm_frac_at_algorithmic_bytes": enc["bytes_per_launch"] / (enc["avg_launch_ms"] / 1e3) / (HBM_PEAK_GBS * 1e9),
        },
        "cpu_baseline": cpu,
        "extra": {"encode_per_layer_launches": enc["per_layer_launches"],
                  "encode_separate_launches": enc["separate_launches"], **extras},
        "vecs_per_s": enc["vecs_per_s"],
    }
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
