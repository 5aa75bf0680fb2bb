"""Allocation-free decode attention (jkv_decode_attention_noalloc) through the
C ABI: identical outputs to jkv_decode_attention on the same inputs, on two
calls in a row (the second smaller, so stale partials of the first would
show), and an argument error beyond the scratch capacity."""

from __future__ import annotations

import pytest
import torch

from jointkv_amd import _lib, _ops
from oracle import jointkv_oracle as ref

pytestmark = pytest.mark.gpu


def _inputs(seed, batch, qh, kvh, length, cap, device, groups=16, stages=2):
    # G2 codes by default; groups=1, stages=16/32 gives full-vector R16/R32
    gen = torch.Generator().manual_seed(seed)
    d = 128 // groups
    sig = (1.0, 0.5) if stages == 2 else tuple(0.8 ** s for s in range(stages))
    q = torch.randn(batch, qh, 128, generator=gen).half().to(device)
    kc = torch.randint(0, 256, (batch, kvh, cap, groups, stages), generator=gen, dtype=torch.uint8).to(device)
    vc = torch.randint(0, 256, (batch, kvh, cap, groups, stages), generator=gen, dtype=torch.uint8).to(device)
    kt = ref.synthetic_tables(gen, (kvh * groups, stages, 256, d), sig, stage_axis=1).half().to(device)
    vt = ref.synthetic_tables(gen, (kvh * groups, stages, 256, d), sig, stage_axis=1).half().to(device)
    lengths = torch.randint(max(1, length // 2), length + 1, (batch,), generator=gen, dtype=torch.int32)
    lengths[0] = length
    return q, kc, vc, kt, vt, lengths.to(device)


def _args(q, kc, vc, kt, vt, lengths, window, table, out):
    batch, qh, _d = q.shape
    _b, kvh, cap, groups, stages = kc.shape
    return [q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), cap,
            kt.data_ptr(), vt.data_ptr(), batch, qh, kvh, groups, 128 // groups, stages, 256, lengths.data_ptr(),
            window, table.data_ptr(), int(table.shape[0]), out.data_ptr()]


def _both(device, q, kc, vc, kt, vt, lengths, window):
    lib = _lib.load()
    table = _ops.rope_table(device, 10000.0, int(lengths.max()) + 1)
    stream = _lib.stream_handle(device)
    ref_out = torch.empty_like(q)
    ws_bytes = int(lib.jkv_decode_workspace_bytes(q.shape[0], q.shape[1], 128, window))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    _lib.check(lib.jkv_decode_attention(*_args(q, kc, vc, kt, vt, lengths, window, table, ref_out),
                                        ws.data_ptr(), ws_bytes, stream))
    out = torch.full_like(q, float("nan"))
    _lib.check(lib.jkv_decode_attention_noalloc(*_args(q, kc, vc, kt, vt, lengths, window, table, out), stream))
    torch.cuda.synchronize(device)
    return ref_out, out


def test_noalloc_decode_matches_workspace_decode_on_two_calls(device):
    # config 4's geometry first (B16, GQA 4, 4096-token window), then a smaller
    # call: its fewer splits must not read the first call's partials
    first = _inputs(3, 16, 32, 8, 4096, 4096, device)
    print("noalloc decode call 1: B=16 QH=32 KVH=8 window=4096", flush=True)
    ref_out, out = _both(device, *first, 4096)
    assert torch.equal(out, ref_out)
    second = _inputs(4, 2, 8, 2, 700, 1024, device)
    print("noalloc decode call 2: B=2 QH=8 KVH=2 window=1024", flush=True)
    ref_out, out = _both(device, *second, 1024)
    assert torch.equal(out, ref_out)
    # and the result is the reference's attention (oracle, 2e-3)
    q, kc, vc, kt, vt, lengths = (t.cpu() for t in second)
    for b in range(2):
        L = int(lengths[b])
        pos = torch.arange(max(0, L - 1024), L)
        khat = ref.frozen_decode(kc[b : b + 1, :, pos % 1024].contiguous(), kt.float(), 2, torch.float16)
        vhat = ref.frozen_decode(vc[b : b + 1, :, pos % 1024].contiguous(), vt.float(), 2, torch.float16)
        expect = ref.decode_attention(q[b : b + 1, :, None], khat, vhat, L - 1, pos)
        err = float((out[b : b + 1].cpu().float() - expect[:, :, 0].float()).abs().max())
        assert err <= 2e-3, f"batch {b}: {err}"


def test_noalloc_decode_full_vector_codes(device):
    # the full-vector (R16 / R32) kernels through the same scratch: 256-token
    # splits, a larger call, then a smaller one with fewer splits
    print("noalloc decode R16: B=4 QH=32 KVH=8 window=1024", flush=True)
    first = _inputs(7, 4, 32, 8, 1024, 1024, device, groups=1, stages=16)
    ref_out, out = _both(device, *first, 1024)
    assert torch.equal(out, ref_out)
    print("noalloc decode R32: B=1 QH=8 KVH=2 window=300", flush=True)
    second = _inputs(8, 1, 8, 2, 290, 512, device, groups=1, stages=32)
    ref_out, out = _both(device, *second, 300)
    assert torch.equal(out, ref_out)


def test_noalloc_decode_sizes_partials_by_the_kernel_it_runs(device):
    # 64 sequences x 32 heads x a 4096-token window: the conservative query
    # (256-token splits) says 17 MB, beyond the 16 MiB scratch, but the
    # group-dim-8 kernel takes 2048-token splits and writes 2.1 MB, so the
    # call is served, with the workspace entry point's bits
    lib = _lib.load()
    cap_bytes = int(lib.jkv_decode_noalloc_max_workspace_bytes())
    assert int(lib.jkv_decode_workspace_bytes(64, 32, 128, 4096)) > cap_bytes
    print("noalloc decode between the old and new limits: B=64 QH=32 KVH=8 window=4096", flush=True)
    ref_out, out = _both(device, *_inputs(6, 64, 32, 8, 4096, 4096, device), 4096)
    assert torch.equal(out, ref_out)


def test_noalloc_decode_rejects_calls_beyond_its_scratch(device):
    lib = _lib.load()
    cap_bytes = int(lib.jkv_decode_noalloc_max_workspace_bytes())
    assert cap_bytes == 16 << 20
    # 256 sequences x 64 heads x a 4096-token window need 2 splits x 130
    # floats each on the group-dim-8 kernel: 17 MB
    q, kc, vc, kt, vt, lengths = _inputs(5, 256, 64, 8, 8, 4096, device)
    table = _ops.rope_table(device, 10000.0, 16)
    out = torch.empty_like(q)
    rc = lib.jkv_decode_attention_noalloc(*_args(q, kc, vc, kt, vt, lengths, 4096, table, out),
                                          _lib.stream_handle(device))
    assert rc == _lib.JKV_EINVAL
    assert b"allocation-free decode attention holds at most" in lib.jkv_last_error()
