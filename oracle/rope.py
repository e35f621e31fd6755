"""Oracle restatement of the reference RoPE helpers (``cb/rope.py:9-89``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Every arithmetic step is the same torch fp32 operation, in the same order, as
the reference, so that on the same torch build the tables are bit-identical.

Parity pinned by: golden tables written from the reference
(``tests/golden/rope_tables.safetensors``: positions {0, 1, 4095, 32767,
40959}, theta {1e4, 1e6}, plus a YaRN configuration), the identity/round-trip
properties of ``cb/rope.py`` exercised by ``tests/test_mapper.py:53-105`` of
the reference, and the closed form cos^2 + sin^2 = magnitude^2.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor


def rotate_half(value: Tensor) -> Tensor:
    """``cb/rope.py:9-13``: split-half rotation ``cat(-x2, x1)``."""
    width = value.shape[-1]
    if width % 2:
        raise ValueError("RoPE head dimension must be even")
    half = width // 2
    return torch.cat((-value[..., half:], value[..., :half]), dim=-1)


def _yarn_bounds(head_dim: int, theta: float, original: int, rotations: float) -> float:
    """``cb/rope.py:46-51``: correction dimension for a rotation count."""
    return head_dim * math.log(original / (rotations * 2 * math.pi)) / (2 * math.log(theta))


def inverse_frequency(
    head_dim: int, theta: float, scaling: dict | None, device="cpu"
) -> tuple[Tensor, float]:
    """``cb/rope.py:28-69``: per-pair inverse frequency and YaRN magnitude."""
    if head_dim % 2:
        raise ValueError("RoPE head dimension must be even")
    ids = torch.arange(0, head_dim, 2, device=device).float()
    inv = 1.0 / (theta ** (ids / head_dim))
    magnitude = 1.0
    if scaling is None:
        return inv, magnitude
    kind = scaling.get("rope_type", scaling.get("type"))
    if kind != "yarn":
        raise ValueError(f"unsupported RoPE scaling type: {kind!r}")
    factor = float(scaling["factor"])
    original = int(scaling["original_max_position_embeddings"])
    fast = float(scaling.get("beta_fast", 32))
    slow = float(scaling.get("beta_slow", 1))
    extrapolation = float(scaling.get("extrapolation_factor", 1))
    attention = float(scaling.get("attn_factor", 1))
    if factor <= 1 or original <= 0:
        raise ValueError(
            "YaRN factor must exceed one and original window must be positive"
        )
    low = max(math.floor(_yarn_bounds(head_dim, theta, original, fast)), 0)
    high = min(math.ceil(_yarn_bounds(head_dim, theta, original, slow)), head_dim - 1)
    if low == high:
        high += 0.001
    ramp = torch.clamp(
        (torch.arange(head_dim // 2, device=device).float() - low) / (high - low), 0, 1
    )
    mask = (1 - ramp) * extrapolation
    interpolated = inv / factor
    inv = interpolated * (1 - mask) + inv * mask
    magnitude = (0.1 * math.log(factor) + 1.0) * attention
    return inv, magnitude


def qwen_rope(
    positions: Tensor,
    *,
    head_dim: int,
    theta: float,
    scaling: dict | None = None,
    dtype: torch.dtype = torch.float32,
) -> tuple[Tensor, Tensor]:
    """``cb/rope.py:16-72``: ``[tokens, head_dim]`` cos/sin, halves duplicated."""
    inv, magnitude = inverse_frequency(head_dim, theta, scaling, positions.device)
    phase = positions.float().unsqueeze(-1) * inv.unsqueeze(0)
    phase = torch.cat((phase, phase), dim=-1)
    return (phase.cos() * magnitude).to(dtype), (phase.sin() * magnitude).to(dtype)


def _broadcast(table: Tensor, like: Tensor) -> Tensor:
    return table.reshape(1, table.shape[0], 1, table.shape[1]).to(like)


def apply_rope(value: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """``cb/rope.py:75-79``: ``x*cos + rotate_half(x)*sin`` on ``[L, n, H, D]``."""
    c = _broadcast(cos, value)
    s = _broadcast(sin, value)
    return value * c + rotate_half(value) * s


def remove_rope(value: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """``cb/rope.py:82-89``: ``(x*cos - rotate_half(x)*sin) / max(cos^2+sin^2, tiny)``."""
    c = _broadcast(cos, value)
    s = _broadcast(sin, value)
    norm = c.square() + s.square()
    return (value * c - rotate_half(value) * s) / norm.clamp_min(
        torch.finfo(value.dtype).tiny
    )
