"""Thin tensor-level wrappers over the libjkv C ABI.

Each function validates shapes and devices on the host, allocates outputs and
workspaces with the PyTorch caching allocator, and enqueues one library call
on the current HIP stream.  Nothing here computes on the CPU.
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _lib


def _encode_states_strides(states: torch.Tensor) -> tuple[torch.Tensor, tuple[int, int, int]]:
    if states.stride(-1) != 1:
        states = states.contiguous()
    return states, (states.stride(0), states.stride(1), states.stride(2))


def rvq_encode(
    states: torch.Tensor,
    tables: torch.Tensor,
    *,
    groups: int,
    group_dim: int,
    exits: Sequence[int],
    whiteners: torch.Tensor | None = None,
    codes_out: torch.Tensor | None = None,
) -> tuple[list[torch.Tensor], torch.Tensor]:
    """Encode ``states[B,H,T,G*d]`` with fp32 masters ``tables[H*G,S,K,d]``.

    Returns (reconstructions at each requested exit depth in ``exits`` order,
    codes ``[B,H,T,G,S]`` uint8).  ``codes_out`` (optional) is written in
    place: any uint8 ``[B,H,T,G,S]`` view whose ``(G,S)`` block is contiguous,
    e.g. the slots of a code cache.
    """

    device = _lib.require_device(states, tables, whiteners)
    batch, heads, tokens, dim = map(int, states.shape)
    problems, stages, clusters, d = map(int, tables.shape)
    if dim != groups * group_dim or d != group_dim or problems != heads * groups:
        raise ValueError("state and table geometry differs")
    if tables.dtype != torch.float32 or not tables.is_contiguous():
        raise ValueError("encode tables must be contiguous fp32 masters")
    if len(exits) > _lib.MAX_EXITS:
        raise ValueError(f"at most {_lib.MAX_EXITS} exits per call")
    lib = _lib.load()
    states, (sb, sh, st) = _encode_states_strides(states)
    if codes_out is None:
        codes = torch.empty((batch, heads, tokens, groups, stages), dtype=torch.uint8, device=device)
    else:
        codes = codes_out
        if (codes.dtype != torch.uint8 or tuple(codes.shape) != (batch, heads, tokens, groups, stages)
                or codes.stride(-1) != 1 or codes.stride(-2) != stages or codes.device != device):
            raise ValueError("codes_out must be uint8 [B,H,T,G,S] with a contiguous (G,S) block")
    recon = [torch.empty((batch, heads, tokens, dim), dtype=states.dtype, device=device) for _ in exits]
    if whiteners is not None:
        whiteners = whiteners.detach().float().contiguous()
        if tuple(whiteners.shape) != (problems, d, d):
            raise ValueError("assignment whitener has invalid geometry")
    ws_bytes = int(lib.jkv_rvq_encode_workspace_bytes(heads, groups, stages, clusters, d, int(whiteners is not None)))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device) if ws_bytes else None
    depth_arr = _lib.ptr_array(ctypes.c_int32, [int(e) for e in exits])
    recon_arr = _lib.ptr_array(ctypes.c_void_p, [r.data_ptr() for r in recon])
    code = lib.jkv_rvq_encode(
        states.data_ptr(), _lib.dtype_code(states.dtype), batch, heads, tokens, groups, d,
        sb, sh, st, tables.data_ptr(), stages, clusters,
        _lib.ptr(whiteners), codes.data_ptr(),
        codes.stride(0), codes.stride(1), codes.stride(2),
        len(exits), depth_arr, recon_arr,
        _lib.ptr(workspace), ws_bytes, _lib.stream_handle(device),
    )
    _lib.check(code)
    return recon, codes


def rvq_encode_kv(
    key: torch.Tensor,
    value: torch.Tensor,
    key_tables: torch.Tensor,
    value_tables: torch.Tensor,
    *,
    groups: int,
    group_dim: int,
    exits: Sequence[int],
    key_codes_out: torch.Tensor | None = None,
    value_codes_out: torch.Tensor | None = None,
):
    """:func:`rvq_encode` of K and of V (same geometry, no whitener) in one
    call; one launch on the grouped MFMA path.  Returns
    ``(key_recon, key_codes, value_recon, value_codes)``."""

    device = _lib.require_device(key, value, key_tables, value_tables)
    if key.shape != value.shape or key.dtype != value.dtype or key_tables.shape != value_tables.shape:
        raise ValueError("K and V must share their geometry")
    batch, heads, tokens, dim = map(int, key.shape)
    problems, stages, clusters, d = map(int, key_tables.shape)
    if dim != groups * group_dim or d != group_dim or problems != heads * groups:
        raise ValueError("state and table geometry differs")
    for t in (key_tables, value_tables):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("encode tables must be contiguous fp32 masters")
    if len(exits) > _lib.MAX_EXITS:
        raise ValueError(f"at most {_lib.MAX_EXITS} exits per call")
    key, strides = _encode_states_strides(key)
    value, vstrides = _encode_states_strides(value)
    if vstrides != strides:
        key, strides = _encode_states_strides(key.contiguous())
        value, vstrides = _encode_states_strides(value.contiguous())
    codes = []
    for out in (key_codes_out, value_codes_out):
        if out is None:
            out = torch.empty((batch, heads, tokens, groups, stages), dtype=torch.uint8, device=device)
        elif (out.dtype != torch.uint8 or tuple(out.shape) != (batch, heads, tokens, groups, stages)
              or out.stride(-1) != 1 or out.stride(-2) != stages or out.device != device):
            raise ValueError("codes_out must be uint8 [B,H,T,G,S] with a contiguous (G,S) block")
        codes.append(out)
    if codes[0].stride()[:3] != codes[1].stride()[:3]:
        raise ValueError("K and V code outputs must share their strides")
    recon_k = [torch.empty((batch, heads, tokens, dim), dtype=key.dtype, device=device) for _ in exits]
    recon_v = [torch.empty((batch, heads, tokens, dim), dtype=key.dtype, device=device) for _ in exits]
    lib = _lib.load()
    ws_bytes = int(lib.jkv_rvq_encode_workspace_bytes(heads, groups, stages, clusters, d, 0))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device) if ws_bytes else None
    depth_arr = _lib.ptr_array(ctypes.c_int32, [int(e) for e in exits])
    code = lib.jkv_rvq_encode_kv(
        key.data_ptr(), value.data_ptr(), _lib.dtype_code(key.dtype), batch, heads, tokens, groups, d,
        *strides, key_tables.data_ptr(), value_tables.data_ptr(), stages, clusters,
        codes[0].data_ptr(), codes[1].data_ptr(), *codes[0].stride()[:3], len(exits), depth_arr,
        _lib.ptr_array(ctypes.c_void_p, [r.data_ptr() for r in recon_k]),
        _lib.ptr_array(ctypes.c_void_p, [r.data_ptr() for r in recon_v]),
        _lib.ptr(workspace), ws_bytes, _lib.stream_handle(device),
    )
    _lib.check(code)
    return recon_k, codes[0], recon_v, codes[1]


def rvq_encode_many(
    states: Sequence[torch.Tensor],
    tables: Sequence[torch.Tensor],
    *,
    groups: int,
    group_dim: int,
    exits: Sequence[int],
) -> list[tuple[list[torch.Tensor], torch.Tensor]]:
    """:func:`rvq_encode` of every ``states[j]`` with ``tables[j]`` (one
    geometry, no whitener) in one call: the layers of a cache and their K and
    V.  On the grouped MFMA path up to 64 encodes share one launch.  Returns
    ``[(reconstructions in exits order, codes), ...]`` in job order, each
    what :func:`rvq_encode` returns for that job."""

    if len(states) != len(tables):
        raise ValueError("one table set per states tensor")
    if not states:
        return []
    # one pass of checks and one allocation per output kind: a cache's 64
    # tensors are enqueued in well under the launch's own GPU time
    first = states[0]
    device = _lib.require_device(first, tables[0])
    batch, heads, tokens, dim = map(int, first.shape)
    problems, stages, clusters, d = map(int, tables[0].shape)
    if dim != groups * group_dim or d != group_dim or problems != heads * groups:
        raise ValueError("state and table geometry differs")
    if len(exits) > _lib.MAX_EXITS:
        raise ValueError(f"at most {_lib.MAX_EXITS} exits per call")
    xshape, xdtype, tshape = first.shape, first.dtype, tables[0].shape
    strides = first.stride()
    index = first.get_device()
    xs = list(states)
    copied = False
    for j, (x, t) in enumerate(zip(states, tables)):
        if x.shape != xshape or x.dtype != xdtype or t.shape != tshape:
            raise ValueError("every job must share the first job's geometry")
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("encode tables must be contiguous fp32 masters")
        if x.get_device() != index or t.get_device() != index:
            raise ValueError("tensors live on different devices")
        if x.stride() != strides or strides[-1] != 1:
            xs[j] = x.contiguous()
            copied = True
    if copied and any(x.stride() != xs[0].stride() for x in xs):
        xs = [x.contiguous() for x in xs]
    sb, sh, st = xs[0].stride()[:3]
    n = len(xs)
    codes_all = torch.empty((n, batch, heads, tokens, groups, stages), dtype=torch.uint8, device=device)
    recon_all = torch.empty((n, len(exits), batch, heads, tokens, dim), dtype=xdtype, device=device)
    c0, cstep = codes_all.data_ptr(), codes_all.stride(0)
    r0, rstep, estep = recon_all.data_ptr(), recon_all.stride(0) * recon_all.element_size(), \
        recon_all.stride(1) * recon_all.element_size()
    lib = _lib.load()
    ws_bytes = int(lib.jkv_rvq_encode_many_workspace_bytes(n, heads, groups, stages, clusters, d))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device) if ws_bytes else None
    code = lib.jkv_rvq_encode_many(
        n, _lib.ptr_array(ctypes.c_void_p, [x.data_ptr() for x in xs]), _lib.dtype_code(xdtype),
        batch, heads, tokens, groups, d, sb, sh, st,
        _lib.ptr_array(ctypes.c_void_p, [t.data_ptr() for t in tables]), stages, clusters,
        _lib.ptr_array(ctypes.c_void_p, [c0 + j * cstep for j in range(n)]), *codes_all.stride()[1:4],
        len(exits), _lib.ptr_array(ctypes.c_int32, [int(e) for e in exits]),
        _lib.ptr_array(ctypes.c_void_p, [r0 + j * rstep + e * estep for j in range(n) for e in range(len(exits))]),
        _lib.ptr(workspace), ws_bytes, _lib.stream_handle(device),
    )
    _lib.check(code)
    codes = codes_all.unbind(0)
    per_exit = [recon_all[:, e].unbind(0) for e in range(len(exits))]
    return [([pe[j] for pe in per_exit], codes[j]) for j in range(n)]


def nearest_f32(states: torch.Tensor, tables: torch.Tensor) -> torch.Tensor:
    """Nearest fp32 codeword per row: ``states[H,N,D]``, ``tables[H,K,D]``
    (fp32, D <= 128) -> int64 ``[H,N]`` (nested_vq.py:178-215 without
    whiteners)."""

    device = _lib.require_device(states, tables)
    if states.ndim != 3 or tables.ndim != 3:
        raise ValueError("nearest-neighbor inputs must have [H,N,D]/[H,K,D]")
    heads, tokens, dim = map(int, states.shape)
    if int(tables.shape[0]) != heads or int(tables.shape[2]) != dim:
        raise ValueError("nearest-neighbor geometry differs")
    states = states.detach().float().contiguous()
    tables = tables.detach().float().contiguous()
    out = torch.empty((heads, tokens), dtype=torch.int64, device=device)
    _lib.check(_lib.load().jkv_nearest_f32(
        states.data_ptr(), heads, tokens, dim, tables.data_ptr(), int(tables.shape[1]),
        out.data_ptr(), _lib.stream_handle(device)))
    return out


def nearest_topk_f32(states: torch.Tensor, tables: torch.Tensor, candidates: int,
                     excluded: torch.Tensor | None = None) -> torch.Tensor:
    """The ``candidates`` nearest fp32 codewords per row, nearest first:
    ``states[H,N,D]``, ``tables[H,K,D]``, optional ``excluded[H,N]`` ->
    int64 ``[H,N,candidates]`` (nested_vq.py:218-260)."""

    device = _lib.require_device(states, tables, excluded)
    if states.ndim != 3 or tables.ndim != 3:
        raise ValueError("nearest-neighbor inputs must have [H,N,D]/[H,K,D]")
    heads, tokens, dim = map(int, states.shape)
    if int(tables.shape[0]) != heads or int(tables.shape[2]) != dim:
        raise ValueError("nearest-neighbor geometry differs")
    if excluded is not None:
        if tuple(excluded.shape) != (heads, tokens):
            raise ValueError("excluded indices must have [H,N] layout")
        excluded = excluded.to(torch.int64).contiguous()
    states = states.detach().float().contiguous()
    tables = tables.detach().float().contiguous()
    out = torch.empty((heads, tokens, int(candidates)), dtype=torch.int64, device=device)
    _lib.check(_lib.load().jkv_nearest_topk_f32(
        states.data_ptr(), heads, tokens, dim, tables.data_ptr(), int(tables.shape[1]), int(candidates),
        None if excluded is None else excluded.data_ptr(), out.data_ptr(), _lib.stream_handle(device)))
    return out


def gain_shape_sums(rows: torch.Tensor, indices: torch.Tensor, clusters: int, *,
                    weights: torch.Tensor | None = None, with_shapes: bool = True):
    """Per-codeword sums of ``rows[H,N,D]`` fp32 under ``indices[H,N]``:
    ``(shape_sums or None, raw_sums, denominators)``, ``[H,K,D]``, ``[H,K,D]``
    and ``[H,K]`` fp32 (see ``jkv_gain_shape_sums``)."""

    device = _lib.require_device(rows, indices, weights)
    if rows.ndim != 3 or indices.shape != rows.shape[:2]:
        raise ValueError("gain-shape rows/indices must be [H,N,D]/[H,N]")
    heads, tokens, dim = map(int, rows.shape)
    rows = rows.detach().float().contiguous()
    indices = indices.to(torch.int64).contiguous()
    if weights is not None:
        if weights.shape != (heads, tokens):
            raise ValueError("gain-shape weights must be [H,N]")
        weights = weights.detach().float().contiguous()
    shape = torch.empty((heads, clusters, dim), dtype=torch.float32, device=device) if with_shapes else None
    raw = torch.empty((heads, clusters, dim), dtype=torch.float32, device=device)
    den = torch.empty((heads, clusters), dtype=torch.float32, device=device)
    lib = _lib.load()
    ws_bytes = int(lib.jkv_gain_shape_sums_workspace_bytes(heads, tokens, dim, clusters, int(with_shapes)))
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
    _lib.check(lib.jkv_gain_shape_sums(
        rows.data_ptr(), heads, tokens, dim, indices.data_ptr(), _lib.ptr(weights), int(clusters),
        int(with_shapes), _lib.ptr(shape), raw.data_ptr(), den.data_ptr(), _lib.ptr(workspace), ws_bytes,
        _lib.stream_handle(device)))
    return shape, raw, den


def subtract_codewords(residual: torch.Tensor, tables: torch.Tensor, indices: torch.Tensor) -> None:
    """``residual[h,n,:] -= tables[h, indices[h,n], :]`` in place (fp32
    contiguous ``[H,N,D]``; ``tables[H,K,D]``, ``indices[H,N]``)."""

    device = _lib.require_device(residual, tables, indices)
    if (residual.dtype != torch.float32 or not residual.is_contiguous() or residual.ndim != 3
            or tables.ndim != 3 or indices.shape != residual.shape[:2]
            or tables.shape[0] != residual.shape[0] or tables.shape[2] != residual.shape[2]):
        raise ValueError("residual must be contiguous fp32 [H,N,D] with tables [H,K,D] and indices [H,N]")
    heads, tokens, dim = map(int, residual.shape)
    tables = tables.detach().float().contiguous()
    indices = indices.to(torch.int64).contiguous()
    _lib.check(_lib.load().jkv_subtract_codewords(
        residual.data_ptr(), heads, tokens, dim, tables.data_ptr(), int(tables.shape[1]), indices.data_ptr(),
        _lib.stream_handle(device)))


def rvq_decode(
    codes: torch.Tensor,
    tables: torch.Tensor,
    *,
    depth: int,
    dtype: torch.dtype,
) -> torch.Tensor:
    """``codes[B,H,T,G,S]`` + fp32 masters ``tables[H*G,S,K,d]`` -> ``[B,H,T,G*d]``.
    fp16 ``tables`` are taken as the deployed words (``fp16(masters)``): the
    same result, half the table bytes read."""

    device = _lib.require_device(codes, tables)
    batch, heads, tokens, groups, stages = map(int, codes.shape)
    problems, t_stages, clusters, d = map(int, tables.shape)
    if problems != heads * groups or t_stages != stages:
        raise ValueError("code and table geometry differs")
    if codes.dtype != torch.uint8 or codes.stride(-1) != 1 or codes.stride(-2) != stages:
        raise ValueError("codes must be uint8 with a contiguous (G,S) block")
    tables = tables.detach()
    lib = _lib.load()
    entry = lib.jkv_rvq_decode
    if tables.dtype == torch.float16:
        entry = lib.jkv_rvq_decode_f16
        tables = tables.contiguous()
    elif tables.dtype != torch.float32 or not tables.is_contiguous():
        tables = tables.float().contiguous()
    out = torch.empty((batch, heads, tokens, groups * d), dtype=dtype, device=device)
    code = entry(
        codes.data_ptr(), codes.stride(0), codes.stride(1), codes.stride(2),
        batch, heads, tokens, groups, d, tables.data_ptr(), stages, clusters, int(depth),
        out.data_ptr(), _lib.dtype_code(dtype), _lib.stream_handle(device),
    )
    _lib.check(code)
    return out


def rvq_scatter_grad(
    grads: Sequence[torch.Tensor],
    exits: Sequence[int],
    codes: torch.Tensor,
    grad_tables: torch.Tensor,
    *,
    group_dim: int,
    deterministic: bool = False,
) -> None:
    """Accumulate the straight-through codebook gradient into ``grad_tables``."""

    device = _lib.require_device(codes, grad_tables, *grads)
    batch, heads, tokens, groups, stages = map(int, codes.shape)
    problems, t_stages, clusters, d = map(int, grad_tables.shape)
    if problems != heads * groups or t_stages != stages or d != group_dim:
        raise ValueError("code and gradient-table geometry differs")
    if grad_tables.dtype != torch.float32 or not grad_tables.is_contiguous():
        raise ValueError("gradient tables must be contiguous fp32")
    dtype = grads[0].dtype
    grads = [g.to(dtype).contiguous() for g in grads]
    # the kernel loads 8- or 4-element slices with one vector load each, which
    # needs the buffer aligned to the slice (a view may not be)
    align = (8 if d % 8 == 0 else 4) * grads[0].element_size()
    grads = [g if g.data_ptr() % align == 0 else g.clone() for g in grads]
    lib = _lib.load()
    ws_bytes = int(lib.jkv_rvq_scatter_workspace_bytes(
        batch, heads, tokens, groups, d, stages, clusters, _lib.dtype_code(dtype), int(deterministic)))
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
    code = lib.jkv_rvq_scatter_grad(
        len(grads), _lib.ptr_array(ctypes.c_void_p, [g.data_ptr() for g in grads]),
        _lib.dtype_code(dtype), _lib.ptr_array(ctypes.c_int32, [int(e) for e in exits]),
        codes.data_ptr(), codes.stride(0), codes.stride(1), codes.stride(2),
        batch, heads, tokens, groups, d, stages, clusters, grad_tables.data_ptr(),
        int(deterministic), _lib.ptr(workspace), ws_bytes, _lib.stream_handle(device),
    )
    _lib.check(code)


def rvq_scatter_grad_many(
    grads: Sequence[Sequence[torch.Tensor]],
    exits: Sequence[int],
    codes: Sequence[torch.Tensor],
    grad_tables: Sequence[torch.Tensor] | None = None,
    *,
    group_dim: int,
    table_shape: Sequence[int] | None = None,
    accumulate: bool | None = None,
    deterministic: bool = False,
) -> list[torch.Tensor]:
    """:func:`rvq_scatter_grad` for every job ``j`` (``grads[j]`` per exit,
    ``codes[j]``) of one geometry in one call.  Given ``grad_tables``, the
    sums are added into them (``accumulate`` True, the default) or stored
    over whatever they hold (``accumulate=False``); without, fresh fp32
    tables of ``table_shape`` are returned holding the sums alone (no zero
    fill).  fp16 gradients with one exit run up to 64 jobs per launch."""

    if len(grads) != len(codes) or (grad_tables is not None and len(grad_tables) != len(codes)):
        raise ValueError("one gradient list, code tensor and table per job")
    if not codes:
        return []
    device = _lib.require_device(*codes, *(g for gs in grads for g in gs),
                                 *(grad_tables if grad_tables is not None else ()))
    batch, heads, tokens, groups, stages = map(int, codes[0].shape)
    n_exits = len(exits)
    if any(len(gs) != n_exits for gs in grads):
        raise ValueError("every job needs one gradient per exit")
    if grad_tables is None:
        if accumulate:
            raise ValueError("accumulating needs grad_tables")
        accumulate = False
    elif accumulate is None:
        accumulate = True
    if grad_tables is not None:
        shape = tuple(map(int, grad_tables[0].shape))
    else:
        if table_shape is None:
            raise ValueError("fresh gradient tables need table_shape")
        shape = tuple(int(v) for v in table_shape)
    problems, t_stages, clusters, d = shape
    if problems != heads * groups or t_stages != stages or d != group_dim:
        raise ValueError("code and gradient-table geometry differs")
    if grad_tables is not None:
        for t in grad_tables:
            if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != shape:
                raise ValueError("gradient tables must be contiguous fp32 of one shape")
        tables = list(grad_tables)
    else:
        tables = list(torch.empty((len(codes), *shape), dtype=torch.float32, device=device).unbind(0))
    strides = codes[0].stride()[:3]
    for c in codes:
        if tuple(c.shape) != (batch, heads, tokens, groups, stages) or c.dtype != torch.uint8:
            raise ValueError("every job's codes must share the first job's geometry")
        if c.stride()[:3] != strides or c.stride(-1) != 1 or c.stride(-2) != stages:
            raise ValueError("every job's codes must share the first job's strides")
    dtype = grads[0][0].dtype
    align = (8 if d % 8 == 0 else 4) * torch.tensor([], dtype=dtype).element_size()
    flat = []
    for gs in grads:
        for g in gs:
            if g.dtype != dtype or not g.is_contiguous():
                g = g.to(dtype).contiguous()
            flat.append(g if g.data_ptr() % align == 0 else g.clone())
    lib = _lib.load()
    ws_bytes = int(lib.jkv_rvq_scatter_workspace_bytes(
        batch, heads, tokens, groups, d, stages, clusters, _lib.dtype_code(dtype), int(deterministic)))
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
    code = lib.jkv_rvq_scatter_grad_many(
        len(codes), n_exits, _lib.ptr_array(ctypes.c_void_p, [g.data_ptr() for g in flat]),
        _lib.dtype_code(dtype), _lib.ptr_array(ctypes.c_int32, [int(e) for e in exits]),
        _lib.ptr_array(ctypes.c_void_p, [c.data_ptr() for c in codes]), *strides,
        batch, heads, tokens, groups, d, stages, clusters,
        _lib.ptr_array(ctypes.c_void_p, [t.data_ptr() for t in tables]), int(accumulate),
        int(deterministic), _lib.ptr(workspace), ws_bytes, _lib.stream_handle(device),
    )
    _lib.check(code)
    return tables


def sumsq(tensors: Sequence[torch.Tensor]) -> torch.Tensor:
    """fp64 squared L2 norms of fp32 device tensors, as one device tensor."""

    device = _lib.require_device(*tensors)
    flat = [t.detach() for t in tensors]
    for t in flat:
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("norm inputs must be contiguous fp32")
    out = torch.empty(len(flat), dtype=torch.float64, device=device)
    code = _lib.load().jkv_sumsq(
        len(flat), _lib.ptr_array(ctypes.c_void_p, [t.data_ptr() for t in flat]),
        _lib.ptr_array(ctypes.c_int64, [t.numel() for t in flat]),
        out.data_ptr(), _lib.stream_handle(device),
    )
    _lib.check(code)
    return out


def scale_sgd(
    grads: Sequence[torch.Tensor],
    scales: Sequence[float],
    *,
    params: Sequence[torch.Tensor] | None = None,
    lr: float = 0.0,
) -> None:
    """``grad *= scale`` in place and, when ``lr`` is non-zero, ``param -= lr*grad``."""

    device = _lib.require_device(*grads)
    if params is not None and len(params) != len(grads):
        raise ValueError("parameter and gradient lists differ")
    for g in grads:
        if g.dtype != torch.float32 or not g.is_contiguous():
            raise ValueError("gradients must be contiguous fp32")
    if params is not None:
        for p, g in zip(params, grads):
            if p.dtype != torch.float32 or not p.is_contiguous() or p.shape != g.shape:
                raise ValueError("parameters must be contiguous fp32 matching their gradients")
    code = _lib.load().jkv_scale_sgd(
        len(grads),
        None if params is None else _lib.ptr_array(ctypes.c_void_p, [p.data_ptr() for p in params]),
        _lib.ptr_array(ctypes.c_void_p, [g.data_ptr() for g in grads]),
        _lib.ptr_array(ctypes.c_int64, [g.numel() for g in grads]),
        _lib.ptr_array(ctypes.c_float, [float(s) for s in scales]),
        float(lr), _lib.stream_handle(device),
    )
    _lib.check(code)


def f32_to_f16(tensor: torch.Tensor) -> torch.Tensor:
    """The deploy round trip ``tensor.half()`` through the library."""

    device = _lib.require_device(tensor)
    src = tensor.detach()
    if src.dtype != torch.float32 or not src.is_contiguous():
        src = src.float().contiguous()
    out = torch.empty(src.shape, dtype=torch.float16, device=device)
    _lib.check(_lib.load().jkv_f32_to_f16(src.data_ptr(), out.data_ptr(), src.numel(), _lib.stream_handle(device)))
    return out


_ROPE_CACHE: dict[tuple, torch.Tensor] = {}


def rotary_inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """inv_freq = 1 / theta^(arange(0, D, 2) / D), computed in fp32 on the CPU
    exactly as the reference's rotary module does (transformers' default rope
    init behind evaluate_mistral_longbench.py:102,113,117)."""

    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))


def rope_table(device: torch.device, theta: float, n_pos: int) -> torch.Tensor:
    """Cached fp16 rotary table [n_pos', 2, 64] (cos row, sin row per position)
    with n_pos' >= n_pos."""

    key = (str(device), float(theta))
    table = _ROPE_CACHE.get(key)
    if table is not None and table.shape[0] >= n_pos:
        return table
    size = 1 << max(12, (max(n_pos, 1) - 1).bit_length())
    inv = rotary_inv_freq(128, theta).to(device)
    table = torch.empty((size, 2, 64), dtype=torch.float16, device=device)
    _lib.check(_lib.load().jkv_rope_table(inv.data_ptr(), size, table.data_ptr(), _lib.stream_handle(device)))
    _ROPE_CACHE[key] = table
    return table


def decode_attention(
    q: torch.Tensor,
    key_codes: torch.Tensor,
    value_codes: torch.Tensor,
    key_tables16: torch.Tensor,
    value_tables16: torch.Tensor,
    lengths: torch.Tensor,
    *,
    window: int,
    rope_theta: float,
    max_length: int | None = None,
    key_new: torch.Tensor | None = None,
    value_new: torch.Tensor | None = None,
) -> torch.Tensor:
    """One decode step of GQA attention straight from the packed code cache.

    ``q[B,QH,D]`` fp16 (pre-RoPE), codes ``[B,KVH,cap,G,S]`` uint8, fp16
    deployed tables ``[KVH*G,S,K,d]``, ``lengths[B]`` int32 (cache length
    including the new token).  ``max_length`` bounds ``lengths`` (the rotary
    table is sized from it); when omitted it is read from the device, which
    synchronises.  With ``key_new``/``value_new`` (``[B,KVH,128]`` fp16, the
    raw K/V of the token at position ``lengths[b]-1``) the same launch
    encodes that token into its ring slot first (``jkv_decode_attention_append``;
    d = 8 caches).  Returns ``[B,QH,D]`` fp16.
    """

    device = _lib.require_device(q, key_codes, value_codes, key_tables16, value_tables16, lengths)
    if q.dtype != torch.float16 or q.ndim != 3 or q.stride(-1) != 1:
        raise ValueError("decode queries must be fp16 [B,QH,D] with a contiguous last axis")
    batch, qheads, dim = map(int, q.shape)
    if key_codes.shape != value_codes.shape or key_codes.dtype != torch.uint8:
        raise ValueError("key/value code caches differ")
    kb, kvheads, cap, groups, stages = map(int, key_codes.shape)
    if kb != batch:
        raise ValueError("query and cache batch differ")
    for c in (key_codes, value_codes):
        if c.stride(-1) != 1 or c.stride(-2) != stages or c.stride(-3) != groups * stages:
            raise ValueError("code caches need contiguous [cap,G,S] blocks")
    if key_codes.stride() != value_codes.stride():
        raise ValueError("key/value code caches need identical strides")
    problems, t_stages, clusters, d = map(int, key_tables16.shape)
    if key_tables16.shape != value_tables16.shape or problems != kvheads * groups or t_stages != stages:
        raise ValueError("code-cache and codebook geometry differs")
    if key_tables16.dtype != torch.float16 or value_tables16.dtype != torch.float16:
        raise ValueError("decode codebooks must be fp16 deployed tables")
    key_tables16 = key_tables16.contiguous()
    value_tables16 = value_tables16.contiguous()
    if lengths.dtype != torch.int32 or lengths.shape != (batch,):
        raise ValueError("lengths must be int32 [B]")
    lengths = lengths.contiguous()
    if max_length is None:
        max_length = int(lengths.max().item()) if batch else 1
    table = rope_table(device, rope_theta, int(max_length) + 1)
    # no sequence sees more than min(window, max_length) keys, so that span is
    # the kernel's window (same visible set; smaller workspace; a cache may be
    # shorter than the model's window)
    span = max(1, min(int(window), int(max_length)))
    lib = _lib.load()
    out = torch.empty((batch, qheads, dim), dtype=torch.float16, device=device)
    ws_bytes = int(lib.jkv_decode_workspace_bytes(batch, qheads, dim, span))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    if key_new is None and value_new is None:
        code = lib.jkv_decode_attention(
            q.data_ptr(), q.stride(0), q.stride(1), key_codes.data_ptr(), value_codes.data_ptr(),
            key_codes.stride(0), key_codes.stride(1), cap, key_tables16.data_ptr(),
            value_tables16.data_ptr(), batch, qheads, kvheads, groups, d, stages, clusters,
            lengths.data_ptr(), span, table.data_ptr(), int(table.shape[0]), out.data_ptr(),
            workspace.data_ptr(), ws_bytes, _lib.stream_handle(device),
        )
    else:
        if key_new is None or value_new is None:
            raise ValueError("append needs both the new key and the new value")
        _lib.require_device(key_new, value_new)
        for t in (key_new, value_new):
            if t.dtype != torch.float16 or tuple(t.shape) != (batch, kvheads, dim) or t.stride(-1) != 1:
                raise ValueError("appended K/V must be fp16 [B,KVH,128] with a contiguous last axis")
        if key_new.stride() != value_new.stride():
            raise ValueError("appended K and V need identical strides")
        code = lib.jkv_decode_attention_append(
            q.data_ptr(), q.stride(0), q.stride(1), key_new.data_ptr(), value_new.data_ptr(),
            key_new.stride(0), key_new.stride(1), key_codes.data_ptr(), value_codes.data_ptr(),
            key_codes.stride(0), key_codes.stride(1), cap, key_tables16.data_ptr(),
            value_tables16.data_ptr(), batch, qheads, kvheads, groups, d, stages, clusters,
            lengths.data_ptr(), span, table.data_ptr(), int(table.shape[0]), out.data_ptr(),
            workspace.data_ptr(), ws_bytes, _lib.stream_handle(device),
        )
    _lib.check(code)
    return out


def decode_attention_window(
    q: torch.Tensor,
    key_window: torch.Tensor,
    value_window: torch.Tensor,
    lengths: torch.Tensor,
    *,
    window: int,
    rope_theta: float,
    max_length: int | None = None,
) -> torch.Tensor:
    """One decode step of GQA attention over decoded fp16 K̂/V̂ windows.

    ``q[B,QH,128]`` fp16 (pre-RoPE), windows ``[B,KVH,cap,128]`` fp16 (rows
    contiguous) with position p in slot ``p % cap``, ``lengths[B]`` int32
    (cache length including the new token).  Returns ``[B,QH,128]`` fp16.
    """

    device = _lib.require_device(q, key_window, value_window, lengths)
    if q.dtype != torch.float16 or q.ndim != 3 or q.stride(-1) != 1:
        raise ValueError("decode queries must be fp16 [B,QH,D] with a contiguous last axis")
    batch, qheads, dim = map(int, q.shape)
    if key_window.shape != value_window.shape or key_window.dtype != torch.float16 or key_window.ndim != 4:
        raise ValueError("decoded windows must be two fp16 [B,KVH,cap,128] tensors of one shape")
    wb, kvheads, cap, wd = map(int, key_window.shape)
    if wb != batch or wd != dim:
        raise ValueError("query and decoded window geometry differ")
    for w in (key_window, value_window):
        if w.stride(-1) != 1 or w.stride(-2) != dim:
            raise ValueError("decoded windows need contiguous [cap,128] blocks")
    if key_window.stride() != value_window.stride():
        raise ValueError("key/value windows need identical strides")
    if lengths.dtype != torch.int32 or lengths.shape != (batch,):
        raise ValueError("lengths must be int32 [B]")
    lengths = lengths.contiguous()
    if max_length is None:
        max_length = int(lengths.max().item()) if batch else 1
    if int(max_length) > cap and int(window) > cap:
        raise ValueError("a sequence longer than the window ring's capacity needs window <= capacity")
    table = rope_table(device, rope_theta, int(max_length) + 1)
    span = max(1, min(int(window), int(max_length)))
    lib = _lib.load()
    out = torch.empty((batch, qheads, dim), dtype=torch.float16, device=device)
    ws_bytes = int(lib.jkv_decode_workspace_bytes(batch, qheads, dim, span))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    code = lib.jkv_decode_attention_window(
        q.data_ptr(), q.stride(0), q.stride(1), key_window.data_ptr(), value_window.data_ptr(),
        key_window.stride(0), key_window.stride(1), cap, batch, qheads, kvheads, lengths.data_ptr(), span,
        table.data_ptr(), int(table.shape[0]), out.data_ptr(), workspace.data_ptr(), ws_bytes,
        _lib.stream_handle(device),
    )
    _lib.check(code)
    return out


def _prefill_operands(q, key, value_or_grad, start_positions, what):
    device = _lib.require_device(q, key, value_or_grad, start_positions)
    for name, t in (("query", q), ("key", key), (what, value_or_grad)):
        if t.dtype != torch.float16 or t.ndim != 4 or t.shape[-1] != 128 or t.stride(-1) != 1:
            raise ValueError(f"prefill {name} must be fp16 [B,H,T,128] with a contiguous last axis")
    batch, qheads, tokens, _dim = map(int, q.shape)
    if key.shape[0] != batch or key.shape[2] != tokens:
        raise ValueError("prefill query/key/value geometry differs")
    kvheads = int(key.shape[1])
    if qheads % kvheads:
        raise ValueError("query heads must be a multiple of kv heads")
    tensors = []
    for t in (q, key, value_or_grad):
        if any(st % 8 for st in t.stride()[:3]) or t.data_ptr() % 16:
            t = t.contiguous()
        tensors.append(t)
    if start_positions.dtype != torch.int32 or start_positions.shape != (batch,):
        raise ValueError("start_positions must be int32 [B]")
    return device, tensors, start_positions.contiguous(), (batch, qheads, kvheads, tokens)


def prefill_attention(
    q: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    start_positions: torch.Tensor,
    *,
    window: int,
    rope_theta: float,
    max_position: int,
    lse: torch.Tensor | None = None,
) -> torch.Tensor:
    """Causal sliding-window GQA attention of one prefill chunk.

    ``q[B,QH,T,128]``, ``key``/``value`` ``[B,KVH,T,128]`` fp16 pre-RoPE,
    ``start_positions[B]`` int32 (position of each row's first token) and
    ``max_position`` an upper bound of ``start + T - 1`` (sizes the rotary
    table).  Returns ``[B,QH,T,128]`` fp16.  With ``lse`` (fp32 ``[B,QH,T]``
    contiguous) each row's log-sum-exp of its visible scores is written there
    for :func:`prefill_attention_value_grad`.
    """

    if key.shape != value.shape:
        raise ValueError("prefill query/key/value geometry differs")
    device, (q, key, value), start_positions, (batch, qheads, kvheads, tokens) = _prefill_operands(
        q, key, value, start_positions, "value")
    if lse is not None and (lse.dtype != torch.float32 or lse.shape != (batch, qheads, tokens)
                            or not lse.is_contiguous() or lse.device != q.device):
        raise ValueError("lse must be a contiguous fp32 [B,QH,T] tensor on the query's device")
    table = rope_table(device, rope_theta, int(max_position) + 1)
    out = torch.empty((batch, qheads, tokens, 128), dtype=torch.float16, device=device)
    code = _lib.load().jkv_prefill_attention(
        q.data_ptr(), *q.stride()[:3], key.data_ptr(), *key.stride()[:3], value.data_ptr(),
        *value.stride()[:3], batch, qheads, kvheads, tokens, 128, start_positions.data_ptr(),
        int(window), table.data_ptr(), int(table.shape[0]), out.data_ptr(),
        lse.data_ptr() if lse is not None else None, _lib.stream_handle(device),
    )
    _lib.check(code)
    return out


PREFILL_CODE_GEOMETRY = (16, 8, (1, 2), 256)  # groups, group dim, stages, codewords of the fused path


def prefill_codes_supported(key_codes: torch.Tensor, key_tables16: torch.Tensor) -> bool:
    """Whether ``jkv_prefill_attention_codes`` takes this code geometry."""

    groups, d, stages, clusters = PREFILL_CODE_GEOMETRY
    return (key_codes.ndim == 5 and int(key_codes.shape[3]) == groups and int(key_codes.shape[4]) in stages
            and key_tables16.ndim == 4 and int(key_tables16.shape[2]) == clusters
            and int(key_tables16.shape[3]) == d)


def prefill_attention_codes(
    q: torch.Tensor,
    key_codes: torch.Tensor,
    value_codes: torch.Tensor,
    key_tables16: torch.Tensor,
    value_tables16: torch.Tensor,
    start_positions: torch.Tensor,
    *,
    window: int,
    rope_theta: float,
    max_position: int,
    lse: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`prefill_attention` over uint8 codes ``[B,KVH,T,16,S]`` (S 1 or
    2) and fp16 deployed tables ``[KVH*16,S,256,8]``, K̂/V̂ rebuilt inside
    the attention kernel.  Bit-identical to :func:`rvq_decode` at depth S
    followed by :func:`prefill_attention`."""

    device = _lib.require_device(q, key_codes, value_codes, key_tables16, value_tables16, start_positions)
    if key_codes.shape != value_codes.shape or key_codes.dtype != torch.uint8 or value_codes.dtype != torch.uint8:
        raise ValueError("key/value codes must be uint8 of one geometry")
    if key_tables16.shape != value_tables16.shape or not prefill_codes_supported(key_codes, key_tables16):
        raise ValueError("prefill from codes needs [B,KVH,T,16,S<=2] codes and [KVH*16,S,256,8] tables")
    if q.dtype != torch.float16 or q.ndim != 4 or q.shape[-1] != 128 or q.stride(-1) != 1:
        raise ValueError("prefill query must be fp16 [B,H,T,128] with a contiguous last axis")
    batch, qheads, tokens, _dim = map(int, q.shape)
    _b, kvheads, _t, groups, stages = map(int, key_codes.shape)
    if (_b, _t) != (batch, tokens) or qheads % kvheads:
        raise ValueError("prefill query/key/value geometry differs")
    if tuple(key_tables16.shape[:2]) != (kvheads * groups, stages):
        raise ValueError("code and table geometry differs")
    if start_positions.dtype != torch.int32 or start_positions.shape != (batch,):
        raise ValueError("start_positions must be int32 [B]")
    start_positions = start_positions.contiguous()
    if lse is not None and (lse.dtype != torch.float32 or lse.shape != (batch, qheads, tokens)
                            or not lse.is_contiguous() or lse.device != q.device):
        raise ValueError("lse must be a contiguous fp32 [B,QH,T] tensor on the query's device")
    if any(st % 8 for st in q.stride()[:3]) or q.data_ptr() % 16:
        q = q.contiguous()
    codes = []
    for c in (key_codes, value_codes):
        if (c.stride(-1) != 1 or c.stride(-2) != stages or c.stride() != key_codes.stride()
                or any(st % 2 for st in c.stride()[:3]) or c.data_ptr() % 2):
            c = c.contiguous()
        codes.append(c)
    if codes[0].stride() != codes[1].stride():
        codes = [c.contiguous() for c in codes]
    tables = []
    for t in (key_tables16, value_tables16):
        t = t.detach()
        if t.dtype != torch.float16 or not t.is_contiguous() or t.data_ptr() % 16:
            t = t.to(torch.float16).contiguous()
        tables.append(t)
    table = rope_table(device, rope_theta, int(max_position) + 1)
    out = torch.empty((batch, qheads, tokens, 128), dtype=torch.float16, device=device)
    kc, vc = codes
    code = _lib.load().jkv_prefill_attention_codes(
        q.data_ptr(), *q.stride()[:3], kc.data_ptr(), vc.data_ptr(), *kc.stride()[:3], tables[0].data_ptr(),
        tables[1].data_ptr(), batch, qheads, kvheads, tokens, groups, 8, stages, 256,
        start_positions.data_ptr(), int(window), table.data_ptr(), int(table.shape[0]),
        out.data_ptr(), lse.data_ptr() if lse is not None else None, _lib.stream_handle(device),
    )
    _lib.check(code)
    return out


def prefill_attention_backward(
    q: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    out: torch.Tensor,
    d_out: torch.Tensor,
    lse: torch.Tensor,
    start_positions: torch.Tensor,
    *,
    window: int,
    rope_theta: float,
    max_position: int,
    need: tuple[bool, bool, bool] = (True, True, True),
):
    """Gradients of :func:`prefill_attention` with respect to the pre-RoPE
    ``q``, ``key`` and ``value`` (fp32; ``None`` where ``need`` is False),
    from the forward's ``out`` and ``lse`` and the output gradient."""

    if key.shape != value.shape:
        raise ValueError("prefill query/key/value geometry differs")
    device, (q, key, value), start_positions, (batch, qheads, kvheads, tokens) = _prefill_operands(
        q, key, value, start_positions, "value")
    _d, (out, _k, d_out), _s, _g = _prefill_operands(out, key, d_out, start_positions, "output gradient")
    if d_out.shape != q.shape or out.shape != q.shape:
        raise ValueError("the output and its gradient must have the query's shape")
    if lse.dtype != torch.float32 or lse.shape != (batch, qheads, tokens) or not lse.is_contiguous():
        raise ValueError("lse must be a contiguous fp32 [B,QH,T] tensor")
    table = rope_table(device, rope_theta, int(max_position) + 1)
    grads = [torch.empty(shape, dtype=torch.float32, device=device) if want else None
             for want, shape in zip(need, ((batch, qheads, tokens, 128), (batch, kvheads, tokens, 128),
                                           (batch, kvheads, tokens, 128)))]
    lib = _lib.load()
    ws_bytes = int(lib.jkv_prefill_backward_workspace_bytes(batch, qheads, kvheads, tokens, int(window)))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    code = lib.jkv_prefill_attention_backward(
        q.data_ptr(), *q.stride()[:3], key.data_ptr(), *key.stride()[:3], value.data_ptr(), *value.stride()[:3],
        out.data_ptr(), *out.stride()[:3], d_out.data_ptr(), *d_out.stride()[:3], lse.data_ptr(),
        batch, qheads, kvheads, tokens, 128, start_positions.data_ptr(), int(window), table.data_ptr(),
        int(table.shape[0]), *[_lib.ptr(g) for g in grads], workspace.data_ptr(), ws_bytes,
        _lib.stream_handle(device),
    )
    _lib.check(code)
    return tuple(grads)


def prefill_attention_value_grad(
    q: torch.Tensor,
    key: torch.Tensor,
    d_out: torch.Tensor,
    lse: torch.Tensor,
    start_positions: torch.Tensor,
    *,
    window: int,
    rope_theta: float,
    max_position: int,
) -> torch.Tensor:
    """Gradient of :func:`prefill_attention` with respect to ``value``:
    fp32 ``[B,KVH,T,128]`` from ``d_out`` (fp16 ``[B,QH,T,128]``) and the
    forward's ``lse``."""

    device, (q, key, d_out), start_positions, (batch, qheads, kvheads, tokens) = _prefill_operands(
        q, key, d_out, start_positions, "output gradient")
    if d_out.shape != q.shape:
        raise ValueError("the output gradient must have the query's shape")
    if lse.dtype != torch.float32 or lse.shape != (batch, qheads, tokens) or not lse.is_contiguous():
        raise ValueError("lse must be a contiguous fp32 [B,QH,T] tensor")
    table = rope_table(device, rope_theta, int(max_position) + 1)
    d_value = torch.empty((batch, kvheads, tokens, 128), dtype=torch.float32, device=device)
    lib = _lib.load()
    ws_bytes = int(lib.jkv_prefill_value_grad_workspace_bytes(batch, qheads, kvheads, tokens, int(window)))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    code = lib.jkv_prefill_attention_value_grad(
        q.data_ptr(), *q.stride()[:3], key.data_ptr(), *key.stride()[:3], d_out.data_ptr(),
        *d_out.stride()[:3], lse.data_ptr(), batch, qheads, kvheads, tokens, 128,
        start_positions.data_ptr(), int(window), table.data_ptr(), int(table.shape[0]),
        d_value.data_ptr(), workspace.data_ptr(), ws_bytes, _lib.stream_handle(device),
    )
    _lib.check(code)
    return d_value
