"""Mapper artifacts: verify a fitted mapper before it is loaded, then load it.

``verify_descriptor`` keeps the reference's contract for a mapper descriptor
(``cb/artifacts.py:17-81``): the descriptor's ``file_hashes`` must name
exactly ``layer_000 .. layer_{L-1}.safetensors`` and the directory must hold
exactly those files; every file must match its SHA-256; with
``check_tensors`` every layer must have the head-local schema, a distinct,
in-range source-layer support, the declared geometry and finite fp32
coefficients, and the coefficient bytes must add up to
``logical_parameter_bytes``. The error texts are the reference's.

How it is done here: the descriptor is read once into a ``_Descriptor``;
each layer file is checked by ``_check_file`` (hash, then the tensor checks
``_check_schema``, ``_check_support``, ``_coefficient_bytes``) on a small
thread pool, since hashing and safetensors reads release the GIL; the
outcomes are then walked in descriptor order, so the error raised is the one
a file-by-file pass would raise first.

Additions for serving processes that load the same mapper repeatedly:

- ``HashRecord``: a small JSON record, keyed by each file's resolved path,
  size and modification time, of SHA-256 digests already computed, and of
  the coefficient bytes of files whose tensor checks already passed for a
  given geometry, so an unchanged file is neither hashed nor re-checked (a
  changed size or time forces both again, and a digest that differs from the
  descriptor still fails);
- ``load_mapper``: verification, then ``PageMapper`` construction from the
  verified directory (TP head slice as ``cb/mapper.py:59-110``).
"""

from __future__ import annotations

import hashlib
import json
import os
import threading
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path

import torch

_LAYER_TENSORS = frozenset({"selected", "headwise", "k_weight", "k_bias", "v_weight", "v_bias"})
_VERIFY_THREADS = 8


def file_sha256(path) -> str:
    h = hashlib.sha256()
    with Path(path).open("rb") as stream:
        for block in iter(lambda: stream.read(8 * 1024 * 1024), b""):
            h.update(block)
    return h.hexdigest()


class HashRecord:
    """Persistent SHA-256 digests and passed tensor checks, keyed by (resolved path, size, mtime_ns)."""

    def __init__(self, path):
        self.path = Path(path)
        try:
            self.entries = json.loads(self.path.read_text())
        except (OSError, ValueError):
            self.entries = {}
        self.computed = 0
        self._lock = threading.Lock()

    @staticmethod
    def _key(p: Path) -> str:
        st = p.stat()
        return f"{p.resolve()}|{st.st_size}|{st.st_mtime_ns}"

    def digest(self, p) -> str:
        p = Path(p)
        key = self._key(p)
        with self._lock:
            value = self.entries.get(key)
        if value is None:
            value = file_sha256(p)
            with self._lock:
                self.entries[key] = value
                self.computed += 1
        return value

    def checked_bytes(self, p, geometry: str) -> int | None:
        """Coefficient bytes of ``p`` if its tensor checks passed for ``geometry``."""
        with self._lock:
            return self.entries.get(f"checked|{geometry}|{self._key(Path(p))}")

    def mark_checked(self, p, geometry: str, nbytes: int) -> None:
        with self._lock:
            self.entries[f"checked|{geometry}|{self._key(Path(p))}"] = int(nbytes)

    def save(self) -> None:
        tmp = self.path.with_suffix(self.path.suffix + ".tmp")
        with self._lock:
            text = json.dumps(self.entries, sort_keys=True)
        tmp.write_text(text)
        os.replace(tmp, self.path)


@dataclass(frozen=True)
class _Descriptor:
    """The fields of a mapper descriptor, with the reference's defaults."""

    path: Path
    root: Path
    mapper_id: str
    layers: int
    source_layers: int
    kv_heads: int
    head_dim: int
    file_hashes: dict
    declared_bytes: int | None
    quality: str

    @classmethod
    def read(cls, path) -> "_Descriptor":
        path = Path(path).expanduser().resolve()
        raw = json.loads(path.read_text())
        root = Path(raw["mapper_dir"])
        if not root.is_absolute():
            root = path.parent / root
        return cls(path=path, root=root.resolve(), mapper_id=raw["mapper_id"],
                   layers=raw.get("target_layers", 64), source_layers=raw.get("source_layers", 40),
                   kv_heads=raw.get("kv_heads", 8), head_dim=raw.get("head_dim", 128),
                   file_hashes=raw["file_hashes"], declared_bytes=raw.get("logical_parameter_bytes"),
                   quality=raw.get("quality", "unmeasured"))

    @property
    def geometry(self) -> str:
        return f"L{self.source_layers}H{self.kv_heads}D{self.head_dim}"

    def check_layer_set(self) -> None:
        want = {f"layer_{i:03d}.safetensors" for i in range(self.layers)}
        present = {p.name for p in self.root.glob("layer_*.safetensors")}
        if set(self.file_hashes) != want or present != want:
            raise ValueError("Missing, extra or noncontiguous mapper layers")


def _check_schema(values: dict) -> None:
    if set(values) != _LAYER_TENSORS or not bool(values["headwise"]):
        raise ValueError("Invalid head-local mapper schema")


def _check_support(selected: torch.Tensor, source_layers: int) -> int:
    """Number of distinct, in-range source layers the layer reads."""
    if selected.ndim != 1 or selected.dtype != torch.int64 or selected.unique().numel() != selected.numel():
        raise ValueError("Invalid source-layer support")
    if selected.numel() == 0 or not (0 <= int(selected.min()) and int(selected.max()) < source_layers):
        raise ValueError("Source-layer support out of range")
    return selected.numel()


def _coefficient_bytes(values: dict, support: int, heads: int, dim: int) -> int:
    total = 0
    for kind in ("k", "v"):
        w, b = values[f"{kind}_weight"], values[f"{kind}_bias"]
        if tuple(w.shape) != (heads, support * dim, dim) or tuple(b.shape) != (heads, dim):
            raise ValueError("Mapper geometry mismatch")
        for t in (w, b):
            if t.dtype != torch.float32 or not bool(torch.isfinite(t).all()):
                raise ValueError("Mapper coefficients must be finite FP32")
            total += t.numel() * t.element_size()
    return total


def _check_file(desc: _Descriptor, name: str, want: str, check_tensors: bool,
                hashes: HashRecord | None) -> tuple[ValueError | None, int]:
    """(the file's first error or None, its coefficient bytes)."""
    p = desc.root / name
    got = hashes.digest(p) if hashes is not None else file_sha256(p)
    if got != want:
        return ValueError(f"Mapper hash mismatch: {name}"), 0
    if not check_tensors:
        return None, 0
    if hashes is not None:
        known = hashes.checked_bytes(p, desc.geometry)
        if known is not None:
            return None, known
    from safetensors.torch import load_file

    values = load_file(str(p))
    try:
        _check_schema(values)
        support = _check_support(values["selected"], desc.source_layers)
        nbytes = _coefficient_bytes(values, support, desc.kv_heads, desc.head_dim)
    except ValueError as error:
        return error, 0
    if hashes is not None:
        hashes.mark_checked(p, desc.geometry, nbytes)
    return None, nbytes


def verify_descriptor(path, *, check_tensors=True, hashes: HashRecord | None = None) -> dict:
    """Check a complete mapper instance before loading its tensors."""
    desc = _Descriptor.read(path)
    desc.check_layer_set()
    names = list(desc.file_hashes.items())
    with ThreadPoolExecutor(max_workers=max(1, min(_VERIFY_THREADS, len(names)))) as pool:
        outcomes = list(pool.map(lambda item: _check_file(desc, *item, check_tensors, hashes), names))
    for error, _ in outcomes:
        if error is not None:
            raise error
    total = sum(nbytes for _, nbytes in outcomes)
    if check_tensors and total != desc.declared_bytes:
        raise ValueError("Logical parameter byte mismatch")
    descriptor_sha256 = hashes.digest(desc.path) if hashes is not None else file_sha256(desc.path)
    if hashes is not None:
        hashes.save()
    return dict(status="passed", mapper_id=desc.mapper_id, mapper_dir=str(desc.root), layers=desc.layers,
                logical_parameter_bytes=total if check_tensors else desc.declared_bytes,
                descriptor_sha256=descriptor_sha256, quality=desc.quality)


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
