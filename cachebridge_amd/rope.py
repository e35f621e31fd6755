"""Split-half RoPE tables for the handoff plan (host side, built once per plan).

The reference computes ``qwen_rope`` per block in fp32 (``cb/rope.py:16-72``):
``inv_freq = 1 / theta^(2i/D)`` (optionally YaRN-blended), ``phase =
float(pos) * inv_freq`` duplicated over both halves, ``cos/sin(phase) *
magnitude``. The plan instead keeps resident ``[positions, D/2]`` fp32 tables
per theta set, built here with the same torch fp32 operations so every entry
has the reference's bits (the two halves of the reference table are equal, so
one half is stored). Tables are evaluated in chunks of at most 32768 elements,
which torch runs on one thread through its vectorized path, so an entry does
not depend on how the range is split.
"""

from __future__ import annotations

import math

import torch

_CHUNK_ELEMENTS = 32768


def _inverse_frequency(head_dim: int, theta: float, scaling: dict | None):
    if head_dim % 2:
        raise ValueError("RoPE head dimension must be even")
    exponents = torch.arange(0, head_dim, 2).float() / head_dim
    inv = 1.0 / (theta ** exponents)
    if scaling is None:
        return inv, 1.0
    rope_type = scaling.get("rope_type", scaling.get("type"))
    if rope_type != "yarn":
        raise ValueError(f"unsupported RoPE scaling type: {rope_type!r}")
    factor = float(scaling["factor"])
    original = int(scaling["original_max_position_embeddings"])
    beta_fast = float(scaling.get("beta_fast", 32))
    beta_slow = float(scaling.get("beta_slow", 1))
    extrapolation = float(scaling.get("extrapolation_factor", 1))
    attn = float(scaling.get("attn_factor", 1))
    if factor <= 1 or original <= 0:
        raise ValueError("YaRN factor must exceed one and original window must be positive")

    def dim_for(rotations: float) -> float:
        return head_dim * math.log(original / (rotations * 2 * math.pi)) / (2 * math.log(theta))

    low = max(math.floor(dim_for(beta_fast)), 0)
    high = min(math.ceil(dim_for(beta_slow)), head_dim - 1)
    if low == high:
        high += 0.001
    ramp = torch.clamp((torch.arange(head_dim // 2).float() - low) / (high - low), 0, 1)
    keep = (1 - ramp) * extrapolation
    inv = (inv / factor) * (1 - keep) + inv * keep
    return inv, (0.1 * math.log(factor) + 1.0) * attn


def rope_tables(head_dim: int, theta: float, scaling: dict | None, positions: int):
    """``(cos, sin)`` of shape ``[positions, head_dim // 2]`` fp32 on the CPU."""
    if positions < 1:
        raise ValueError("positions must be positive")
    inv, magnitude = _inverse_frequency(head_dim, float(theta), scaling)
    half = head_dim // 2
    cos = torch.empty(positions, half)
    sin = torch.empty(positions, half)
    step = max(1, _CHUNK_ELEMENTS // head_dim)
    with torch.inference_mode():
        for p0 in range(0, positions, step):
            pos = torch.arange(p0, min(positions, p0 + step))
            phase = pos.float().unsqueeze(-1) * inv.unsqueeze(0)
            phase = torch.cat((phase, phase), dim=-1)
            cos[p0: p0 + len(pos)] = (phase.cos() * magnitude)[:, :half]
            sin[p0: p0 + len(pos)] = (phase.sin() * magnitude)[:, :half]
    return cos, sin


def qwen_rope(positions: torch.Tensor, *, head_dim: int, theta: float,
              scaling: dict | None = None, dtype: torch.dtype = torch.float32):
    """``[tokens, head_dim]`` split-half cos/sin (API of ``cb/rope.py:16-72``)."""
    inv, magnitude = _inverse_frequency(head_dim, float(theta), scaling)
    phase = positions.float().unsqueeze(-1) * inv.to(positions.device).unsqueeze(0)
    phase = torch.cat((phase, phase), dim=-1)
    return (phase.cos() * magnitude).to(dtype), (phase.sin() * magnitude).to(dtype)


def rotate_half(value: torch.Tensor) -> torch.Tensor:
    """``cat(-x2, x1)`` over the last dimension (``cb/rope.py:9-13``)."""
    if value.shape[-1] % 2:
        raise ValueError("RoPE head dimension must be even")
    a, b = value.chunk(2, dim=-1)
    return torch.cat((-b, a), dim=-1)


def apply_rope(value: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate ``[L, tokens, H, D]`` keys (``cb/rope.py:75-79``)."""
    shape = (1, cos.shape[0], 1, cos.shape[1])
    return value * cos.reshape(shape).to(value) + rotate_half(value) * sin.reshape(shape).to(value)
