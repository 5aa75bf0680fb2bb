"""numpy front end of the fp64 brute-force checker (test infrastructure only)."""

from __future__ import annotations

import ctypes

import numpy as np

from . import build_oracle


def _p(a: np.ndarray) -> int:
    return a.ctypes.data_as(ctypes.c_void_p).value


def rvq_encode(x: np.ndarray, tables: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """x [N,D], tables [S,K,D] -> codes int32 [N,S], best and second distances [N,S]."""

    lib = build_oracle.load()
    x = np.ascontiguousarray(x, dtype=np.float64)
    tables = np.ascontiguousarray(tables, dtype=np.float64)
    n, d = x.shape
    s, k, d2 = tables.shape
    assert d == d2 and d <= 4096
    codes = np.zeros((n, s), dtype=np.int32)
    best = np.zeros((n, s), dtype=np.float64)
    second = np.zeros((n, s), dtype=np.float64)
    lib.bf_rvq_encode(_p(x), _p(tables), n, s, k, d, _p(codes), _p(best), _p(second))
    return codes, best, second


def scatter(g: np.ndarray, codes: np.ndarray, stages: int, clusters: int, depth: int) -> np.ndarray:
    """g [N,D], codes [N,S] -> grad [S,K,D] (fp64)."""

    lib = build_oracle.load()
    g = np.ascontiguousarray(g, dtype=np.float64)
    codes = np.ascontiguousarray(codes, dtype=np.int32)
    n, d = g.shape
    out = np.zeros((stages, clusters, d), dtype=np.float64)
    lib.bf_scatter(_p(g), _p(codes), n, stages, clusters, d, depth, _p(out))
    return out


def attention_row(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    lib = build_oracle.load()
    q = np.ascontiguousarray(q, dtype=np.float64)
    k = np.ascontiguousarray(k, dtype=np.float64)
    v = np.ascontiguousarray(v, dtype=np.float64)
    t, d = k.shape
    out = np.zeros(d, dtype=np.float64)
    lib.bf_attention_row(_p(q), _p(k), _p(v), t, d, _p(out))
    return out
