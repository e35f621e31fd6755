"""GPU: a verified mapper descriptor loads into the same GPU mapper as its directory.

``load_mapper`` verifies the descriptor (hashes, schema, geometry, byte count)
and then builds ``PageMapper`` from the verified directory with the TP head
slice; the result maps a page bit for bit as a directly built mapper does (the
directory mapper itself is held to the oracle by the parity tests). A tampered
file is rejected before anything is loaded.
"""

from __future__ import annotations

import json

import pytest
import torch
from safetensors.torch import save_file

from cachebridge_amd.artifacts import HashRecord, file_sha256, load_mapper
from cachebridge_amd.mapper import PageMapper

pytestmark = pytest.mark.gpu


def _artifact(tmp_path, *, layers=3, heads=4, dim=64, selected=(1, 3), source_layers=4):
    g = torch.Generator().manual_seed(3)
    names, total = {}, 0
    for i in range(layers):
        s = len(selected)
        values = dict(selected=torch.tensor(list(selected)), headwise=torch.tensor(True),
                      k_weight=torch.randn(heads, s * dim, dim, generator=g) / dim,
                      v_weight=torch.randn(heads, s * dim, dim, generator=g) / dim,
                      k_bias=torch.randn(heads, dim, generator=g) * 0.1,
                      v_bias=torch.randn(heads, dim, generator=g) * 0.1)
        total += sum(values[k].numel() * 4 for k in ("k_weight", "v_weight", "k_bias", "v_bias"))
        p = tmp_path / f"layer_{i:03d}.safetensors"
        save_file(values, str(p))
        names[p.name] = file_sha256(p)
    d = dict(mapper_id="gpu-test", mapper_dir=".", target_layers=layers, source_layers=source_layers,
             kv_heads=heads, head_dim=dim, logical_parameter_bytes=total, file_hashes=names)
    manifest = tmp_path / "mapper.json"
    manifest.write_text(json.dumps(d))
    return manifest


@pytest.mark.parametrize("rank,size", [(0, 1), (1, 2)])
def test_verified_load_maps_like_the_directory_mapper(tmp_path, rank, size):
    manifest = _artifact(tmp_path)
    kw = dict(source_rope_theta=1e4, target_rope_theta=1e6, target_tp_rank=rank, target_tp_size=size,
              dtype=torch.bfloat16, max_positions=512)
    mapper, report = load_mapper(manifest, hashes=HashRecord(tmp_path / "hashes.json"), **kw)
    assert report["status"] == "passed" and report["layers"] == 3
    direct = PageMapper(tmp_path, method="cachebridge", **kw)
    local = 4 // size
    g = torch.Generator().manual_seed(5)
    page = torch.randn(2, 4, 96, local, 64, generator=g).to(torch.bfloat16)
    a = mapper.map_page(page, position_start=7, source_head_offset=rank * local, output_device="cuda")
    b = direct.map_page(page, position_start=7, source_head_offset=rank * local, output_device="cuda")
    torch.cuda.synchronize()
    assert a.shape == (2, 3, 96, local, 64)
    assert torch.equal(a, b)


def test_tampered_artifact_is_never_loaded(tmp_path):
    manifest = _artifact(tmp_path)
    p = tmp_path / "layer_001.safetensors"
    p.write_bytes(p.read_bytes() + b"!")
    with pytest.raises(ValueError, match="hash mismatch"):
        load_mapper(manifest, source_rope_theta=1e4, target_rope_theta=1e6, max_positions=512)
