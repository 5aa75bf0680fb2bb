"""Readers and writers for the reference's codebook artifacts.

* Parent codebook layers ``layer_XX.pt``, one per decoder layer, as
  ``make_codec`` reads them (experiments_followup_mistral/
  train_mistral_v_only.py:54-79):
  * gsrq cells: ``{"codebooks": {"key": [8,S,256,128], "value": ...},
    "key_assignment_whiteners": [8,128,128] | None}`` with S = 16 (gsrq1) or
    32 (gsrq2);
  * cq cells: ``{"key": {"codebooks": [8,G,256,d], "selector_whiteners":
    [8,G,d,d] | None}, "value": {"codebooks": ...}}`` with (G, d) = (16, 8)
    (cq1) or (32, 4) (cq2); a missing selector is the identity.
* V-only exports ``value_layer_XX.pt`` (written at train_mistral_v_only.py:
  168-172, read back at evaluate_mistral_longbench.py:147-150):
  ``{"layer": int, "value_table": fp16 tensor, "identity": dict}``, listed
  in the run receipt as ``{"path", "sha256", "bytes"}`` rows.

Files are read with ``torch.load(..., weights_only=True)``: plain dicts of
tensors, numbers and strings load; anything that would need arbitrary
unpickling is refused with the loader's own error.
"""

from __future__ import annotations

import hashlib
from pathlib import Path
from typing import Any

import torch

from .cq_tac import ClosedLoopGroupedCQ
from .uniform_depth_tac import ClosedLoopUniformResidualVQ

#: (stages or groups, 256, d) per cell, as make_codec asserts them
CELL_GEOMETRY = {
    "gsrq1": (16, 256, 128),
    "gsrq2": (32, 256, 128),
    "cq1": (16, 256, 8),
    "cq2": (32, 256, 4),
}


def sha256_file(path: str | Path) -> str:
    """Hex SHA-256 of a file, read in 1 MiB blocks (train_mistral_v_only.py:32-37)."""

    digest = hashlib.sha256()
    with Path(path).open("rb") as handle:
        for block in iter(lambda: handle.read(1 << 20), b""):
            digest.update(block)
    return digest.hexdigest()


def load_artifact(path: str | Path) -> Any:
    """``torch.load`` restricted to tensors and plain containers."""

    return torch.load(Path(path), map_location="cpu", weights_only=True)


def _atomic_save(value: Any, target: Path) -> None:
    # train_mistral_v_only.py:40-44: write beside the target, then rename
    target.parent.mkdir(parents=True, exist_ok=True)
    temporary = target.with_suffix(target.suffix + ".tmp")
    torch.save(value, temporary)
    temporary.replace(target)


def make_codec(cell: str, source: str | Path, *, layers: int = 32, device: torch.device | str = "cuda"):
    """The codec ``make_codec`` builds from a parent directory
    (train_mistral_v_only.py:54-79): fp16 codebooks per layer become the
    codec's fp32 masters; gsrq cells keep their key assignment whiteners,
    cq cells their selector whiteners (identity when absent)."""

    if cell not in CELL_GEOMETRY:
        raise ValueError(f"unknown codebook cell {cell!r}")
    source = Path(source)
    keys, values, selectors = [], [], []
    for layer in range(layers):
        body = load_artifact(source / f"layer_{layer:02d}.pt")
        if cell.startswith("gsrq"):
            key = body["codebooks"]["key"].half().contiguous()
            value = body["codebooks"]["value"].half().contiguous()
            selectors.append(body.get("key_assignment_whiteners"))
        else:
            key = body["key"]["codebooks"].half().contiguous()
            value = body["value"]["codebooks"].half().contiguous()
            selector = body["key"].get("selector_whiteners")
            if selector is None:
                selector = torch.eye(key.shape[-1]).repeat(key.shape[0], key.shape[1], 1, 1)
            selectors.append(selector)
        if tuple(key.shape) != (key.shape[0], *CELL_GEOMETRY[cell]):
            raise ValueError(f"layer {layer}: {cell} codebooks have shape {tuple(key.shape)}")
        if key.shape != value.shape:
            raise ValueError(f"layer {layer}: key and value codebooks differ")
        keys.append(key)
        values.append(value)
    rate = 1.0 if cell.endswith("1") else 2.0
    if cell.startswith("gsrq"):
        codec = ClosedLoopUniformResidualVQ(keys, values, selectors, depth=keys[0].shape[1], dynamic_bpa=rate,
                                            token_chunk_size=1024)
    else:
        codec = ClosedLoopGroupedCQ(keys, values, selectors, dynamic_bpa=rate, token_chunk_size=64)
    return codec.to(device)


def save_value_layers(codec, output: str | Path, identity: dict) -> list[dict]:
    """Write ``value_layer_XX.pt`` per layer as the V-only run exports them
    (train_mistral_v_only.py:164-172) and return the receipt rows."""

    output = Path(output)
    rows = []
    for layer, table in enumerate(codec.value_tables):
        path = output / f"value_layer_{layer:02d}.pt"
        _atomic_save({"layer": layer, "value_table": table.detach().half().cpu().contiguous(),
                      "identity": identity}, path)
        rows.append({"path": str(path), "sha256": sha256_file(path), "bytes": path.stat().st_size})
    return rows


def load_value_layers(codec, value_layer_files: list[dict]) -> None:
    """Copy exported V tables into ``codec`` after checking each file's
    SHA-256 against its receipt row (evaluate_mistral_longbench.py:145-150)."""

    if len(value_layer_files) != len(codec.value_tables):
        raise ValueError("the receipt lists a different number of value layers")
    for layer, item in enumerate(value_layer_files):
        path = Path(item["path"])
        if sha256_file(path) != item["sha256"]:
            raise ValueError(f"value layer {layer}: SHA-256 differs from the receipt")
        body = load_artifact(path)
        if int(body["layer"]) != layer:
            raise ValueError(f"{path.name} holds layer {body['layer']}, expected {layer}")
        target = codec.value_tables[layer]
        table = body["value_table"]
        if tuple(table.shape) != tuple(target.shape):
            raise ValueError(f"value layer {layer}: table shape {tuple(table.shape)} differs from the codec's")
        with torch.no_grad():
            target.copy_(table.to(device=target.device, dtype=target.dtype))
