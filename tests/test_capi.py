"""C ABI checks that need no GPU: exports, signatures, argument validation."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from jointkv_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "jkv.h"


def _declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(jkv_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_function():
    lib = _lib.load()
    declared = _declared_functions()
    assert "jkv_rvq_encode" in declared and "jkv_decode_attention" in declared
    for name in declared:
        assert hasattr(lib, name), f"libjkv.so does not export {name}"
    assert declared == set(_lib.SIGNATURES), "ctypes signatures out of sync with include/jkv.h"


def test_version_and_error_text():
    lib = _lib.load()
    assert lib.jkv_version() >= 100
    assert isinstance(lib.jkv_last_error(), bytes)


def _encode_call(**overrides):
    lib = _lib.load()
    args = dict(states=1, dtype=0, B=1, H=1, T=4, G=1, d=8, sb=32, sh=32, st=8, tables=1, S=1, K=256,
                whiteners=None, codes=1, cb=4, ch=4, ct=1, n_exits=0, exits=None, recon=None,
                ws=None, ws_bytes=0, stream=None)
    args.update(overrides)
    return lib.jkv_rvq_encode(*args.values())


def test_encode_rejects_invalid_geometry_before_touching_the_device():
    # These return before any HIP call, so they run without a GPU.
    assert _encode_call(K=300) == _lib.JKV_EINVAL
    assert b"256" in _lib.load().jkv_last_error()
    assert _encode_call(d=0) == _lib.JKV_EINVAL
    assert _encode_call(dtype=7) == _lib.JKV_EINVAL
    assert _encode_call(d=200) == _lib.JKV_EINVAL
    depths = (ctypes.c_int32 * 1)(5)
    assert _encode_call(n_exits=1, exits=depths, S=2) == _lib.JKV_EINVAL
    assert b"ladder" in _lib.load().jkv_last_error()
    # an empty problem is a successful no-op
    assert _encode_call(T=0) == _lib.JKV_OK


def test_workspace_queries():
    lib = _lib.load()
    assert lib.jkv_rvq_encode_workspace_bytes(8, 16, 2, 256, 8, 0) == 0
    assert lib.jkv_rvq_encode_workspace_bytes(8, 16, 2, 256, 8, 1) == 8 * 16 * 2 * 256 * 8 * 4
    # full-vector codebooks: fp16 tables + -|c|^2/2 plane + partial max norms per (head, stage)
    assert lib.jkv_rvq_encode_workspace_bytes(8, 1, 2, 256, 128, 0) == 8 * 2 * (256 * 128 * 2 + 256 * 4 + 64)
    assert lib.jkv_rvq_encode_workspace_bytes(8, 1, 33, 256, 128, 0) == 0
    assert lib.jkv_rvq_encode_workspace_bytes(8, 1, 2, 128, 128, 0) == 0
    # whitened full-vector: plus M c per codeword (fp32), M and its hi/lo planes per head
    assert lib.jkv_rvq_encode_workspace_bytes(8, 1, 2, 256, 128, 1) == (
        8 * 2 * (256 * 128 * 2 + 256 * 4 + 64) + 8 * 2 * 256 * 128 * 4 + 8 * (128 * 128 * 4 + 256 * 128 * 2))
    # whitened elsewhere: fp32 selector tables
    assert lib.jkv_rvq_encode_workspace_bytes(8, 16, 2, 256, 8, 1) == 8 * 16 * 2 * 256 * 8 * 4
    F16, BF16 = _lib.JKV_F16, _lib.JKV_BF16
    bins = 8 * 16 * 2 * 256 * 8  # [H*G,S,K,d] of the config-5 V codebooks
    # one chunk of rows: bins go straight into the gradient
    assert lib.jkv_rvq_scatter_workspace_bytes(1, 8, 512, 16, 8, 2, 256, F16, 0) == 0
    # fp16 sums are exact (fixed point), so a deterministic request needs nothing more
    assert lib.jkv_rvq_scatter_workspace_bytes(1, 8, 512, 16, 8, 2, 256, F16, 1) == 0
    # bf16 deterministic: ordered partials per 256-row chunk
    assert lib.jkv_rvq_scatter_workspace_bytes(1, 8, 512, 16, 8, 2, 256, BF16, 1) == 2 * bins * 4
    # fp16, 8-dim groups at config 5: one block per (head, group, stage)
    # already fills the chip (256 blocks), so no row chunks and no partials
    assert lib.jkv_rvq_scatter_workspace_bytes(4, 8, 2048, 16, 8, 2, 256, F16, 0) == 0
    # one stage: one block per (head, group) holds the bins, 128 blocks take
    # 2 row chunks of 4096 rows with 64-bit partials
    assert lib.jkv_rvq_scatter_workspace_bytes(4, 8, 2048, 16, 8, 1, 256, F16, 0) == bins * 8
    # bf16 (fp32 bins): one block per (head, group, stage, 8 dims) already fills the chip
    assert lib.jkv_rvq_scatter_workspace_bytes(4, 8, 2048, 16, 8, 2, 256, BF16, 0) == 0
    assert lib.jkv_rvq_scatter_workspace_bytes(4, 8, 2048, 1, 128, 2, 256, F16, 0) == 0
    # one head: 32 blocks, so 4 row chunks of 2048 rows with per-chunk partials,
    # 64-bit for fixed point and 32-bit otherwise
    head = 16 * 2 * 256 * 8
    assert lib.jkv_rvq_scatter_workspace_bytes(4, 1, 2048, 16, 8, 2, 256, F16, 0) == 4 * head * 8
    assert lib.jkv_rvq_scatter_workspace_bytes(4, 1, 2048, 16, 8, 2, 256, _lib.JKV_F32, 0) == 4 * head * 4
    # d not a multiple of 4: global atomics, no workspace
    assert lib.jkv_rvq_scatter_workspace_bytes(4, 1, 2048, 1, 6, 2, 256, F16, 0) == 0
    assert lib.jkv_decode_workspace_bytes(16, 32, 128, 4096) == 16 * 32 * 16 * 130 * 4


def test_decode_rejects_unsupported_geometry():
    # Only argument combinations that fail validation: a valid geometry with
    # placeholder pointers would launch a kernel.
    lib = _lib.load()
    rc = lib.jkv_decode_attention(1, 0, 0, 1, 1, 0, 0, 4096, 1, 1, 1, 32, 8, 8, 8, 2, 256, 1,
                                  4096, 1, 8192, 1, 1, 1 << 30, None)
    assert rc == _lib.JKV_EINVAL and b"head_dim" in lib.jkv_last_error()
    rc = lib.jkv_decode_attention(1, 0, 0, 1, 1, 0, 0, 100, 1, 1, 1, 32, 8, 16, 8, 2, 256, 1,
                                  4096, 1, 8192, 1, 1, 1 << 30, None)
    assert rc == _lib.JKV_EINVAL and b"capacity" in lib.jkv_last_error()
    rc = lib.jkv_decode_attention(1, 0, 0, 1, 1, 0, 0, 4096, 1, 1, 1, 32, 8, 16, 8, 2, 256, 1,
                                  4096, 1, 0, 1, 1, 1 << 30, None)
    assert rc == _lib.JKV_EINVAL and b"rotary" in lib.jkv_last_error()


def test_decode_window_rejects_bad_arguments():
    # validation only: every call below fails before a launch
    lib = _lib.load()
    # capacity below the window
    rc = lib.jkv_decode_attention_window(1, 0, 0, 16, 16, 0, 0, 100, 1, 32, 8, 1, 4096, 1, 8192, 1, 1,
                                         1 << 30, None)
    assert rc == _lib.JKV_EINVAL and b"capacity" in lib.jkv_last_error()
    # rows not 16-byte aligned
    rc = lib.jkv_decode_attention_window(1, 0, 0, 18, 16, 0, 0, 4096, 1, 32, 8, 1, 4096, 1, 8192, 1, 1,
                                         1 << 30, None)
    assert rc == _lib.JKV_EINVAL and b"aligned" in lib.jkv_last_error()
    # GQA group of 3 query heads
    rc = lib.jkv_decode_attention_window(1, 0, 0, 16, 16, 0, 0, 4096, 1, 24, 8, 1, 4096, 1, 8192, 1, 1,
                                         1 << 30, None)
    assert rc == _lib.JKV_EINVAL and b"GQA" in lib.jkv_last_error()
    # workspace too small
    rc = lib.jkv_decode_attention_window(1, 0, 0, 16, 16, 0, 0, 4096, 1, 32, 8, 1, 4096, 1, 8192, 1, 1,
                                         16, None)
    assert rc == _lib.JKV_EINVAL and b"workspace" in lib.jkv_last_error()


def test_scatter_rejects_misaligned_deterministic_gradients():
    # Validation fails before any launch: the gradient pointer (2) is not
    # aligned to an 8-element fp16 slice and a deterministic sum was asked for.
    lib = _lib.load()
    grads = _lib.ptr_array(ctypes.c_void_p, [2])
    depths = _lib.ptr_array(ctypes.c_int32, [2])
    rc = lib.jkv_rvq_scatter_grad(1, grads, _lib.JKV_F16, depths, 1, 512, 256, 32, 1, 8, 8, 16,
                                  8, 2, 256, 1, 1, None, 0, None)
    assert rc == _lib.JKV_EINVAL and b"aligned" in lib.jkv_last_error()


def test_product_rejects_host_tensors_loudly():
    import jointkv_amd as jkv

    states = torch.randn(1, 2, 4, 8)
    tables = torch.randn(2, 1, 256, 8)
    with pytest.raises(ValueError, match="HIP"):
        jkv.hard_residual_vq_exits(states, tables, prefixes=(1,))


def test_nearest_rejects_rows_beyond_the_grid_before_touching_the_device():
    # one 256-thread block per 64 rows: 2^30 rows would need a 2^32-item grid
    lib = _lib.load()
    dummy = ctypes.c_void_p(16)
    for name, extra in (("jkv_nearest_f32", []), ("jkv_nearest_topk_f32", [ctypes.c_int64(2), ctypes.c_void_p(0)])):
        fn = getattr(lib, name)
        args = [dummy, ctypes.c_int64(1), ctypes.c_int64(1 << 30), ctypes.c_int64(8), dummy, ctypes.c_int64(256)]
        args += extra + [dummy, ctypes.c_void_p(0)]
        assert fn(*args) == _lib.JKV_EINVAL
        assert b"rows per head" in lib.jkv_last_error()


def test_many_job_entry_points_validate_before_touching_the_device():
    # argument errors and empty calls return before any HIP call
    lib = _lib.load()
    p = (ctypes.c_void_p * 1)(16)
    depth = (ctypes.c_int32 * 1)(1)
    bad_depth = (ctypes.c_int32 * 1)(3)
    enc = dict(n=1, states=p, dtype=0, B=1, H=1, T=4, G=1, d=8, sb=32, sh=32, st=8, tables=p, S=1, K=256,
               codes=p, cb=4, ch=4, ct=1, n_exits=1, exits=depth, recon=None, ws=None, ws_bytes=0, stream=None)

    def encode_many(**kw):
        a = dict(enc)
        a.update(kw)
        return lib.jkv_rvq_encode_many(*a.values())

    assert encode_many(n=-1) == _lib.JKV_EINVAL
    assert encode_many(K=0) == _lib.JKV_EINVAL
    assert encode_many(n_exits=99) == _lib.JKV_EINVAL
    assert encode_many(n=0) == _lib.JKV_OK
    assert encode_many(T=0) == _lib.JKV_OK
    assert encode_many(states=None) == _lib.JKV_EINVAL
    assert encode_many(exits=bad_depth) == _lib.JKV_EINVAL
    assert b"ladder" in lib.jkv_last_error()

    sc = dict(n=1, n_exits=1, grads=p, dtype=0, exits=depth, codes=p, cb=4, ch=4, ct=2, B=1, H=1, T=4, G=1,
              d=8, S=2, K=256, tables=p, accumulate=1, deterministic=0, ws=None, ws_bytes=0, stream=None)

    def scatter_many(**kw):
        a = dict(sc)
        a.update(kw)
        return lib.jkv_rvq_scatter_grad_many(*a.values())

    assert scatter_many(n=-1) == _lib.JKV_EINVAL
    assert scatter_many(K=300) == _lib.JKV_EINVAL
    assert scatter_many(dtype=7) == _lib.JKV_EINVAL
    assert scatter_many(n_exits=0) == _lib.JKV_EINVAL
    assert scatter_many(n=0) == _lib.JKV_OK
    assert scatter_many(codes=None) == _lib.JKV_EINVAL
    assert scatter_many(exits=bad_depth) == _lib.JKV_EINVAL
    # an empty problem that accumulates is a no-op
    assert scatter_many(T=0) == _lib.JKV_OK


def test_many_job_wrappers_reject_host_tensors_and_accept_empty_lists():
    from jointkv_amd import _ops

    assert _ops.rvq_encode_many([], [], groups=1, group_dim=8, exits=(1,)) == []
    assert _ops.rvq_scatter_grad_many([], (1,), [], group_dim=8) == []
    with pytest.raises(ValueError, match="HIP"):
        _ops.rvq_encode_many([torch.randn(1, 2, 4, 8).half()], [torch.randn(2, 1, 256, 8)], groups=1,
                             group_dim=8, exits=(1,))
    with pytest.raises(ValueError, match="HIP"):
        _ops.rvq_scatter_grad_many([[torch.randn(1, 2, 4, 8).half()]], (1,),
                                   [torch.zeros(1, 2, 4, 1, 1, dtype=torch.uint8)], group_dim=8,
                                   table_shape=(2, 1, 256, 8))
