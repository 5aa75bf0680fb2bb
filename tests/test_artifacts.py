"""Reference artifact formats: parent codebook layers and V-only exports
(host only, CPU)."""

from __future__ import annotations

import pickle

import pytest
import torch

from jointkv_amd import artifacts


def _gsrq_parent(tmp_path, layers, stages, heads=2, whitener=True, seed=0):
    gen = torch.Generator().manual_seed(seed)
    tmp_path.mkdir(parents=True, exist_ok=True)
    bodies = []
    for layer in range(layers):
        body = {
            "codebooks": {
                "key": torch.randn(heads, stages, 256, 128, generator=gen).half(),
                "value": torch.randn(heads, stages, 256, 128, generator=gen).half(),
            },
            "key_assignment_whiteners": torch.randn(heads, 128, 128, generator=gen) if whitener else None,
        }
        torch.save(body, tmp_path / f"layer_{layer:02d}.pt")
        bodies.append(body)
    return bodies


def test_gsrq_parent_builds_the_reference_codec(tmp_path):
    bodies = _gsrq_parent(tmp_path, layers=2, stages=16)
    codec = artifacts.make_codec("gsrq1", tmp_path, layers=2, device="cpu")
    assert codec.depth == 16 and codec.dynamic_bpa == 1.0 and codec.token_chunk_size == 1024
    for layer, body in enumerate(bodies):
        assert torch.equal(codec.key_tables[layer].data, body["codebooks"]["key"].float())
        assert torch.equal(codec.value_tables[layer].data, body["codebooks"]["value"].float())
        assert not codec.key_tables[layer].requires_grad and codec.value_tables[layer].requires_grad
        assert torch.equal(codec.whitener(layer), body["key_assignment_whiteners"])


def test_cq_parent_without_selector_gets_the_identity(tmp_path):
    gen = torch.Generator().manual_seed(1)
    for layer in range(2):
        torch.save({"key": {"codebooks": torch.randn(2, 32, 256, 4, generator=gen).half()},
                    "value": {"codebooks": torch.randn(2, 32, 256, 4, generator=gen).half()}},
                   tmp_path / f"layer_{layer:02d}.pt")
    codec = artifacts.make_codec("cq2", tmp_path, layers=2, device="cpu")
    assert codec.dynamic_bpa == 2.0 and codec.token_chunk_size == 64
    assert codec.key_tables[0].shape == (2, 32, 256, 4)


def test_wrong_cell_geometry_is_refused(tmp_path):
    _gsrq_parent(tmp_path, layers=1, stages=16, whitener=False)
    with pytest.raises(ValueError, match="gsrq2 codebooks"):
        artifacts.make_codec("gsrq2", tmp_path, layers=1, device="cpu")
    with pytest.raises(ValueError, match="unknown codebook cell"):
        artifacts.make_codec("gsrq3", tmp_path, layers=1, device="cpu")


def test_value_layers_round_trip_with_receipt(tmp_path):
    _gsrq_parent(tmp_path / "parent", layers=2, stages=16, whitener=False)
    codec = artifacts.make_codec("gsrq1", tmp_path / "parent", layers=2, device="cpu")
    with torch.no_grad():
        for p in codec.value_tables:
            p.add_(0.125)
    identity = {"endpoint": "test", "parent_layer_sha256": ["a", "b"]}
    rows = artifacts.save_value_layers(codec, tmp_path / "run", identity)
    assert [r["path"].endswith(f"value_layer_{i:02d}.pt") for i, r in enumerate(rows)] == [True, True]
    body = artifacts.load_artifact(rows[1]["path"])
    assert body["layer"] == 1 and body["identity"] == identity
    assert body["value_table"].dtype == torch.float16 and body["value_table"].is_contiguous()
    fresh = artifacts.make_codec("gsrq1", tmp_path / "parent", layers=2, device="cpu")
    artifacts.load_value_layers(fresh, rows)
    for a, b in zip(fresh.value_tables, codec.value_tables):
        assert torch.equal(a.data, b.data.half().float())
    # a file that no longer matches its receipt row is refused
    torch.save({"layer": 0, "value_table": torch.zeros(2, 16, 256, 128).half(), "identity": identity},
               rows[0]["path"])
    with pytest.raises(ValueError, match="SHA-256"):
        artifacts.load_value_layers(fresh, rows)


class _Opaque:
    pass


def test_loader_refuses_pickled_objects(tmp_path):
    path = tmp_path / "layer_00.pt"
    torch.save({"codebooks": _Opaque()}, path)
    with pytest.raises(pickle.UnpicklingError):
        artifacts.load_artifact(path)
