"""Mapper descriptors: an incomplete or modified mapper fails before use (CPU).

Restates the reference's ``tests/test_artifacts.py:10-60`` against
``cachebridge_amd.artifacts.verify_descriptor`` and adds the hash record:
unchanged files are not hashed twice, changed ones are.
"""

from __future__ import annotations

import json

import pytest
import torch
from safetensors.torch import save_file

from cachebridge_amd import artifacts
from cachebridge_amd.artifacts import HashRecord, file_sha256, verify_descriptor


def fixture(tmp_path, layers=1):
    names = {}
    for i in range(layers):
        values = dict(selected=torch.tensor([0]), headwise=torch.tensor(True), k_weight=torch.eye(2)[None],
                      v_weight=torch.eye(2)[None], k_bias=torch.zeros(1, 2), v_bias=torch.zeros(1, 2))
        p = tmp_path / f"layer_{i:03d}.safetensors"
        save_file(values, str(p))
        names[p.name] = file_sha256(p)
    d = dict(mapper_id="test", mapper_dir=".", target_layers=layers, source_layers=1, kv_heads=1, head_dim=2,
             logical_parameter_bytes=48 * layers, file_hashes=names)
    manifest = tmp_path / "mapper.json"
    manifest.write_text(json.dumps(d))
    return manifest, tmp_path / "layer_000.safetensors", d


def test_verified_portable_descriptor(tmp_path):
    manifest, _, _ = fixture(tmp_path)
    report = verify_descriptor(manifest)
    assert report["layers"] == 1 and report["status"] == "passed" and report["logical_parameter_bytes"] == 48


def test_changed_coefficients_rejected(tmp_path):
    manifest, path, _ = fixture(tmp_path)
    path.write_bytes(path.read_bytes() + b"changed")
    with pytest.raises(ValueError, match="hash mismatch"):
        verify_descriptor(manifest)


def test_missing_layer_rejected(tmp_path):
    manifest, path, _ = fixture(tmp_path)
    path.unlink()
    with pytest.raises(ValueError, match="Missing"):
        verify_descriptor(manifest)


def test_extra_layer_rejected(tmp_path):
    manifest, path, _ = fixture(tmp_path)
    (tmp_path / "layer_001.safetensors").write_bytes(path.read_bytes())
    with pytest.raises(ValueError, match="Missing"):
        verify_descriptor(manifest)


def test_schema_and_byte_count_rejected(tmp_path):
    manifest, path, d = fixture(tmp_path)
    d["logical_parameter_bytes"] = 47
    manifest.write_text(json.dumps(d))
    with pytest.raises(ValueError, match="byte mismatch"):
        verify_descriptor(manifest)
    bad = dict(selected=torch.tensor([0, 0]), headwise=torch.tensor(True), k_weight=torch.eye(2)[None],
               v_weight=torch.eye(2)[None], k_bias=torch.zeros(1, 2), v_bias=torch.zeros(1, 2))
    save_file(bad, str(path))
    d["file_hashes"][path.name] = file_sha256(path)
    manifest.write_text(json.dumps(d))
    with pytest.raises(ValueError, match="support"):
        verify_descriptor(manifest)


def test_hash_record_skips_unchanged_files_and_catches_changes(tmp_path, monkeypatch):
    manifest, path, _ = fixture(tmp_path, layers=3)
    record_path = tmp_path / "hashes.json"
    calls = []
    real = artifacts.file_sha256
    monkeypatch.setattr(artifacts, "file_sha256", lambda p: calls.append(str(p)) or real(p))
    verify_descriptor(manifest, hashes=HashRecord(record_path))
    assert len(calls) == 4  # three layers and the descriptor
    calls.clear()
    second = HashRecord(record_path)
    verify_descriptor(manifest, hashes=second)
    assert calls == [] and second.computed == 0
    path.write_bytes(path.read_bytes() + b"x")  # new size: hashed again, and rejected
    with pytest.raises(ValueError, match="hash mismatch"):
        verify_descriptor(manifest, hashes=HashRecord(record_path))
    assert any(c.endswith("layer_000.safetensors") for c in calls)


def test_hash_record_skips_tensor_checks_of_unchanged_files(tmp_path, monkeypatch):
    import safetensors.torch as st

    manifest, path, _ = fixture(tmp_path, layers=3)
    record_path = tmp_path / "hashes.json"
    assert verify_descriptor(manifest, hashes=HashRecord(record_path))["logical_parameter_bytes"] == 144
    loads = []
    real = st.load_file
    monkeypatch.setattr(st, "load_file", lambda p, *a, **k: loads.append(p) or real(p, *a, **k))
    report = verify_descriptor(manifest, hashes=HashRecord(record_path))
    assert loads == [] and report["logical_parameter_bytes"] == 144
    # a changed file is hashed and checked again (here: it no longer matches its digest)
    path.write_bytes(path.read_bytes() + b"x")
    with pytest.raises(ValueError, match="hash mismatch"):
        verify_descriptor(manifest, hashes=HashRecord(record_path))


def test_first_failing_layer_in_descriptor_order_is_reported(tmp_path):
    manifest, _, d = fixture(tmp_path, layers=4)
    for i in (1, 3):
        p = tmp_path / f"layer_{i:03d}.safetensors"
        p.write_bytes(p.read_bytes() + b"!")
    with pytest.raises(ValueError, match="hash mismatch: layer_001"):
        verify_descriptor(manifest)
