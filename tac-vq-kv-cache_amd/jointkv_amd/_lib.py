"""ctypes binding of ``libjkv.so`` (the C ABI declared in ``include/jkv.h``).

The library is the only compute path of this package: there is no CPU or
pure-PyTorch fallback.  Loading fails loudly when the shared object is
missing, and every operator checks that its tensors live on a HIP device.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("JKV_LIB", _HERE / "libjkv.so"))

JKV_OK = 0
JKV_EINVAL = -1
JKV_EHIP = -2
JKV_ENOTSUP = -3
JKV_F16, JKV_BF16, JKV_F32 = 0, 1, 2
MAX_EXITS = 8

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/jkv.h one for one.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "jkv_version": (ctypes.c_int, []),
    "jkv_last_error": (ctypes.c_char_p, []),
    "jkv_rvq_encode_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i32]),
    "jkv_rvq_encode": (
        ctypes.c_int,
        [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp,
         _i64, _i64, _i64, _i32, _vp, _vp, _vp, _i64, _vp],
    ),
    "jkv_rvq_encode_kv": (
        ctypes.c_int,
        [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp,
         _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _i64, _vp],
    ),
    "jkv_rvq_encode_many_workspace_bytes": (_i64, [_i32, _i64, _i64, _i64, _i64, _i64]),
    "jkv_rvq_encode_many": (
        ctypes.c_int,
        [_i32, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _vp,
         _i64, _i64, _i64, _i32, _vp, _vp, _vp, _i64, _vp],
    ),
    "jkv_nearest_f32": (ctypes.c_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp]),
    "jkv_nearest_topk_f32": (ctypes.c_int, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp]),
    "jkv_gain_shape_sums": (
        ctypes.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _i64, _vp]),
    "jkv_gain_shape_sums_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i32]),
    "jkv_subtract_codewords": (ctypes.c_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp]),
    "jkv_rvq_decode": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _vp, _i32,
         _vp],
    ),
    "jkv_rvq_decode_f16": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _vp, _i32,
         _vp],
    ),
    "jkv_rvq_scatter_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32]),
    "jkv_rvq_scatter_grad": (
        ctypes.c_int,
        [_i32, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _vp, _i32, _vp, _i64, _vp],
    ),
    "jkv_rvq_scatter_grad_many": (
        ctypes.c_int,
        [_i32, _i32, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _vp, _i32, _i32, _vp, _i64, _vp],
    ),
    "jkv_pair_block_select": (
        ctypes.c_int,
        [_vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp,
         _vp],
    ),
    "jkv_sumsq": (ctypes.c_int, [_i32, _vp, _vp, _vp, _vp]),
    "jkv_scale_sgd": (ctypes.c_int, [_i32, _vp, _vp, _vp, _vp, _f32, _vp]),
    "jkv_decode_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "jkv_decode_attention": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp],
    ),
    "jkv_decode_attention_append": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp],
    ),
    "jkv_decode_noalloc_max_workspace_bytes": (_i64, []),
    "jkv_decode_attention_noalloc": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _vp, _i64, _vp, _i64, _vp, _vp],
    ),
    "jkv_decode_attention_window": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp,
         _i64, _vp],
    ),
    "jkv_prefill_attention": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp],
    ),
    "jkv_prefill_attention_codes": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp],
    ),
    "jkv_prefill_attention_value_grad": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
         _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp],
    ),
    "jkv_prefill_value_grad_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "jkv_prefill_attention_backward": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
         _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp,
         _vp, _i64, _vp],
    ),
    "jkv_prefill_backward_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "jkv_prefill_attention_key_grad": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
         _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp],
    ),
    "jkv_rope_table": (ctypes.c_int, [_vp, _i64, _vp, _vp]),
    "jkv_f32_to_f16": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
}

_lib: ctypes.CDLL | None = None


class JKVError(RuntimeError):
    """A HIP runtime or launch failure reported by libjkv."""


def load() -> ctypes.CDLL:
    """Load ``libjkv.so`` once and declare every entry point's signature."""

    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.is_file():
        raise ImportError(
            f"libjkv.so not found at {LIB_PATH}; build it with "
            "`python tac-vq-kv-cache_amd/build_lib.py` (gfx950 HIP kernels are the only "
            "compute path of jointkv_amd)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def check(code: int) -> None:
    """Map a libjkv return code to the reference's exception types."""

    if code == JKV_OK:
        return
    lib = load()
    message = lib.jkv_last_error().decode(errors="replace")
    if code in (JKV_EINVAL, JKV_ENOTSUP):
        raise ValueError(message)
    raise JKVError(message)


def stream_handle(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must share one HIP device; returns it."""

    device = None
    for tensor in tensors:
        if tensor is None:
            continue
        if tensor.device.type != "cuda":
            raise ValueError(
                "jointkv_amd runs on the MI355X (HIP) device only; got a tensor on "
                f"{tensor.device}"
            )
        if device is None:
            device = tensor.device
        elif tensor.device != device:
            raise ValueError("tensors live on different devices")
    if device is None:
        raise ValueError("no device tensor given")
    return device


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return JKV_F16
    if dtype == torch.bfloat16:
        return JKV_BF16
    if dtype == torch.float32:
        return JKV_F32
    raise ValueError(f"unsupported dtype {dtype}")


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else int(tensor.data_ptr())


def ptr_array(ctype, values) -> ctypes.Array:
    return (ctype * max(1, len(values)))(*values)
