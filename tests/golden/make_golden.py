"""Write the golden fixtures of the hot path (inputs and expected outputs).

The reference repository holds no tensors (its tests draw tiny seeded
``torch.randn`` inputs), so the fixtures here are produced by this build's
oracle (``oracle/jointkv_oracle.py``, the eager-PyTorch restatement of the
reference's op sequence) on seeded inputs of the BASELINE geometries, scaled
down.  Each ``.npz`` holds plain arrays (no pickles); ``tests/test_golden.py``
checks that the oracle still reproduces them and the GPU tests check the HIP
path against them.

Usage: python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import jointkv_oracle as ref  # noqa: E402


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy()


def g2_encode(gen: torch.Generator) -> dict:
    """GSRQ-2 grouped residual VQ (config 2 geometry, 2 heads x 64 tokens)."""

    states = ref.synthetic_states(gen, 1, 2, 64)
    tables = ref.synthetic_tables(gen, (2, 16, 2, 256, 8), (1.0, 0.5), stage_axis=2)
    exits, codes, d1, d2 = ref.grouped_residual_vq(states, tables, prefixes=(1, 2), return_margins=True)
    return {
        "states": _np(states),
        "tables_f16": _np(tables.half()),
        "codes": _np(codes),
        "exit1": _np(exits[1]),
        "exit2": _np(exits[2]),
        "d1": _np(d1),
        "d2": _np(d2),
    }


def cq2_encode(gen: torch.Generator) -> dict:
    """Reference cq2 grouped CQ ([H,32,256,4], config 3 geometry)."""

    states = ref.synthetic_states(gen, 1, 2, 64)
    books = ref.synthetic_tables(gen, (2, 32, 256, 4), (1.0,), stage_axis=0)
    recon, codes, d1, d2 = ref.hard_grouped_cq(states, books, return_margins=True)
    return {
        "states": _np(states),
        "books_f16": _np(books.half()),
        "codes": _np(codes),
        "recon": _np(recon),
        "d1": _np(d1),
        "d2": _np(d2),
    }


def scatter(gen: torch.Generator, g2: dict) -> dict:
    """STE codebook gradient of the first 16 tokens of the G2 fixture, as the
    non-zero bins (the gradient of an unused codeword is exactly zero)."""

    codes = torch.from_numpy(g2["codes"][:, :, :16].copy())
    upstream = (torch.randn(1, 2, 16, 128, generator=gen) * 1e-3 ** 0.5).half()
    grad = ref.table_gradient([upstream], [2], codes, (32, 2, 256, 8), accumulate=torch.float64).float()
    flat = grad.reshape(32 * 2 * 256, 8)
    rows = torch.nonzero(flat.abs().sum(dim=1) > 0).flatten()
    return {
        "codes": _np(codes),
        "upstream": _np(upstream),
        "bin_index": _np(rows.to(torch.int32)),
        "bin_value": _np(flat[rows]),
    }


def decode(gen: torch.Generator, g2: dict) -> dict:
    """One decode step over an 80-token G2 code cache (GQA 4, 2 kv heads),
    K codebooks = the G2 fixture's tables, V codebooks = half of them."""

    kt = torch.from_numpy(g2["tables_f16"]).reshape(32, 2, 256, 8)
    vt = (kt.float() * 0.5).half()
    length = 80
    kc = torch.randint(0, 256, (1, 2, length, 16, 2), generator=gen, dtype=torch.uint8)
    vc = torch.randint(0, 256, (1, 2, length, 16, 2), generator=gen, dtype=torch.uint8)
    q = torch.randn(1, 8, 1, 128, generator=gen).half()
    khat = ref.frozen_decode(kc, kt.float(), 2, torch.float16)
    vhat = ref.frozen_decode(vc, vt.float(), 2, torch.float16)
    out = ref.decode_attention(q, khat, vhat, length - 1, torch.arange(length))
    return {"q": _np(q), "k_codes": _np(kc), "v_codes": _np(vc), "out": _np(out)}


def prefill(gen: torch.Generator) -> dict:
    """A 24-token prefill chunk at positions 100.. (GQA 4, window 16)."""

    q = torch.randn(1, 8, 24, 128, generator=gen).half()
    k = torch.randn(1, 2, 24, 128, generator=gen).half()
    v = torch.randn(1, 2, 24, 128, generator=gen).half()
    out = ref.prefill_attention(q, k, v, (100,), window=16)
    return {"q": _np(q), "k": _np(k), "v": _np(v), "start": np.array([100], dtype=np.int32),
            "window": np.array(16, dtype=np.int64), "out": _np(out)}


def clip(gen: torch.Generator) -> dict:
    """Global and per_layer_kv clipping of two layers' V gradients."""

    grads = [torch.randn(2, 2, 64, 8, generator=gen) * 0.05, torch.randn(2, 2, 64, 8, generator=gen) * 0.02]
    out = {"g0": _np(grads[0]), "g1": _np(grads[1])}
    for mode in ("global", "per_layer_kv"):
        tables = [torch.zeros(2, 2, 64, 8, requires_grad=True) for _ in grads]
        for t, g in zip(tables, grads):
            t.grad = g.clone()
        audit = ref.clip_codebook_gradients([], tables, maximum_norm=0.5, mode=mode)
        out[f"{mode}_g0"] = _np(tables[0].grad)
        out[f"{mode}_g1"] = _np(tables[1].grad)
        out[f"{mode}_norm_before"] = np.array(audit["total_norm_before_clip"], dtype=np.float64)
    return out


def main() -> None:
    gen = torch.Generator().manual_seed(8601)
    g2 = g2_encode(gen)
    fixtures = {
        "g2_encode": g2,
        "cq2_encode": cq2_encode(gen),
        "scatter": scatter(gen, g2),
        "decode": decode(gen, g2),
        "prefill": prefill(gen),
        "clip": clip(gen),
    }
    for name, arrays in fixtures.items():
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **arrays)
        print(f"wrote {path.name}: {path.stat().st_size / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
