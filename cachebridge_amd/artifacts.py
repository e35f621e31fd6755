"""Mapper artifacts: verify a fitted mapper before it is loaded, then load it.

``verify_descriptor`` keeps the reference's contract for a mapper descriptor
(``cb/artifacts.py:17-81``): the descriptor's ``file_hashes`` must name
exactly ``layer_000 .. layer_{L-1}.safetensors`` and the directory must hold
exactly those files; every file must match its SHA-256; with
``check_tensors`` every layer must have the head-local schema, a distinct,
in-range source-layer support, the declared geometry and finite fp32
coefficients, and the coefficient bytes must add up to
``logical_parameter_bytes``.

Two additions for serving processes that load the same mapper repeatedly:

- ``HashRecord``: a small JSON record, keyed by each file's resolved path,
  size and modification time, of SHA-256 digests already computed, so an
  unchanged file is not hashed again (a changed size or time forces a new
  hash, and a digest that differs from the descriptor still fails);
- ``load_mapper``: verification, then ``PageMapper`` construction from the
  verified directory (TP head slice as ``cb/mapper.py:59-110``).
"""

from __future__ import annotations

import hashlib
import json
import os
from pathlib import Path

import torch


def file_sha256(path) -> str:
    h = hashlib.sha256()
    with Path(path).open("rb") as stream:
        for block in iter(lambda: stream.read(8 * 1024 * 1024), b""):
            h.update(block)
    return h.hexdigest()


class HashRecord:
    """Persistent SHA-256 digests keyed by (resolved path, size, mtime_ns)."""

    def __init__(self, path):
        self.path = Path(path)
        try:
            self.entries = json.loads(self.path.read_text())
        except (OSError, ValueError):
            self.entries = {}
        self.computed = 0

    @staticmethod
    def _key(p: Path) -> str:
        st = p.stat()
        return f"{p.resolve()}|{st.st_size}|{st.st_mtime_ns}"

    def digest(self, p) -> str:
        p = Path(p)
        key = self._key(p)
        value = self.entries.get(key)
        if value is None:
            value = file_sha256(p)
            self.entries[key] = value
            self.computed += 1
        return value

    def save(self) -> None:
        tmp = self.path.with_suffix(self.path.suffix + ".tmp")
        tmp.write_text(json.dumps(self.entries, sort_keys=True))
        os.replace(tmp, self.path)


def verify_descriptor(path, *, check_tensors=True, hashes: HashRecord | None = None) -> dict:
    """Check a complete mapper instance before loading its tensors."""
    path = Path(path).expanduser().resolve()
    d = json.loads(path.read_text())
    root = Path(d["mapper_dir"])
    root = root.resolve() if root.is_absolute() else (path.parent / root).resolve()
    depth = d.get("target_layers", 64)
    expected = {f"layer_{i:03d}.safetensors" for i in range(depth)}
    if set(d["file_hashes"]) != expected or {p.name for p in root.glob("layer_*.safetensors")} != expected:
        raise ValueError("Missing, extra or noncontiguous mapper layers")
    digest = hashes.digest if hashes is not None else file_sha256
    tensor_bytes = 0
    if check_tensors:
        from safetensors.torch import load_file
    for name, want in d["file_hashes"].items():
        p = root / name
        if digest(p) != want:
            raise ValueError(f"Mapper hash mismatch: {name}")
        if not check_tensors:
            continue
        values = load_file(str(p))
        if set(values) != {"selected", "headwise", "k_weight", "k_bias", "v_weight", "v_bias"} \
                or not bool(values["headwise"]):
            raise ValueError("Invalid head-local mapper schema")
        selected = values["selected"]
        if selected.ndim != 1 or selected.dtype != torch.int64 or len(set(selected.tolist())) != len(selected):
            raise ValueError("Invalid source-layer support")
        if selected.numel() == 0 or int(selected.min()) < 0 or int(selected.max()) >= d.get("source_layers", 40):
            raise ValueError("Source-layer support out of range")
        heads, dim = d.get("kv_heads", 8), d.get("head_dim", 128)
        for kind in ("k", "v"):
            w, b = values[kind + "_weight"], values[kind + "_bias"]
            if w.shape != (heads, len(selected) * dim, dim) or b.shape != (heads, dim):
                raise ValueError("Mapper geometry mismatch")
            if (w.dtype != torch.float32 or b.dtype != torch.float32 or not torch.isfinite(w).all()
                    or not torch.isfinite(b).all()):
                raise ValueError("Mapper coefficients must be finite FP32")
            tensor_bytes += w.numel() * w.element_size() + b.numel() * b.element_size()
    if check_tensors and tensor_bytes != d["logical_parameter_bytes"]:
        raise ValueError("Logical parameter byte mismatch")
    descriptor_sha256 = digest(path)
    if hashes is not None:
        hashes.save()
    return dict(status="passed", mapper_id=d["mapper_id"], mapper_dir=str(root), layers=depth,
                logical_parameter_bytes=tensor_bytes if check_tensors else d["logical_parameter_bytes"],
                descriptor_sha256=descriptor_sha256, quality=d.get("quality", "unmeasured"))


def load_mapper(descriptor, *, source_rope_theta, target_rope_theta, source_rope_scaling=None,
                target_rope_scaling=None, device="cuda", target_tp_rank=0, target_tp_size=1,
                hashes: HashRecord | None = None, check_tensors=True, **kwargs):
    """Verify ``descriptor``, then build the GPU ``PageMapper`` from its directory.

    Returns ``(mapper, report)``; nothing is loaded when verification fails.
    """
    from .mapper import PageMapper

    report = verify_descriptor(descriptor, check_tensors=check_tensors, hashes=hashes)
    mapper = PageMapper(report["mapper_dir"], method="cachebridge", source_rope_theta=source_rope_theta,
                        target_rope_theta=target_rope_theta, source_rope_scaling=source_rope_scaling,
                        target_rope_scaling=target_rope_scaling, device=device,
                        target_tp_rank=target_tp_rank, target_tp_size=target_tp_size, **kwargs)
    return mapper, report
