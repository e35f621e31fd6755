"""Structured-state installs on either side of the handoff (Gemma 3, Qwen3.5).

The install contracts are the reference's (same functions, arguments, errors
and messages): ``materialize_kv`` / ``install_kv`` for the Gemma 3
local/global cache roster (``cb/architectures/gemma3.py:38-94``);
``required_replay``, ``install_attention_kv`` and ``install_linear_state``
for Qwen3.5 (``cb/architectures/qwen35.py:64-160``). Every install is
all-or-nothing: nothing in the cache changes unless every check passed.

How it is done here: a target cache layer is first given a role
(``_role``: full or sliding attention, linear attention, or neither) from the
methods it has; each install's checks are a lazy generator of problems
(``_*_problems``) in the reference's order, and the install raises the first
one, or, if there is none, performs its writes. The retained window of a
Gemma layer comes from ``layouts.retained_window``, the same function the
mapper's windowed install uses.

``transform_delta_state`` maps Qwen3.5 DeltaNet memory as ``A^T U B``
(``cb/architectures/qwen35.py:52-61``) with the HIP kernel behind
``cb_delta_state_transform`` (16x16x4 fp32 / fp64 MFMAs). Inputs must be GPU
tensors; there is no CPU path.

Paths are relative to the reference repository; ``cb/`` = ``src/cachebridge/``.
"""

from __future__ import annotations

from collections.abc import Iterator
from dataclasses import dataclass

import torch

from . import _lib
from .layouts import retained_window


def _positive_int(value, name: str) -> int:
    if type(value) is not int or value < 1:
        raise ValueError(f"{name} must be a positive integer")
    return value


def _raise_first(problems: Iterator[Exception]) -> None:
    problem = next(problems, None)
    if problem is not None:
        raise problem


_LINEAR_LAYER_API = ("update_conv_state", "update_recurrent_state", "has_previous_state",
                     "recurrent_states", "conv_states")


def _role(layer) -> str:
    """``"linear"``, ``"sliding"``, ``"full"`` or ``"other"`` for a cache layer (duck-typed).

    A layer with recurrent state is never an attention layer; an attention
    layer must accept ``update(key, value)``.
    """
    if all(hasattr(layer, name) for name in _LINEAR_LAYER_API):
        return "linear"
    if hasattr(layer, "recurrent_states") or not hasattr(layer, "update"):
        return "other"
    return "sliding" if getattr(layer, "is_sliding", False) else "full"


def _kv_pair_problem(key, value) -> Exception | None:
    if key.ndim != 4 or key.shape != value.shape or key.dtype != value.dtype or key.device != value.device:
        return ValueError("K/V must match [batch,heads,tokens,head_dim], dtype and device")
    return None


# ---------------------------------------------------------------------------
# Gemma 3 (cb/architectures/gemma3.py)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class MaterializedKV:
    """Retained content-space history of one Gemma layer (``gemma3.py:31-36``)."""

    key: torch.Tensor
    value: torch.Tensor
    first_position: int
    prefix_length: int


def materialize_kv(content_key, value, *, layer_type, sliding_window, prefix_length=None):
    """Keep what a Gemma layer attends to: the last ``min(T, W - 1)`` tokens of
    a sliding layer, every token of a global one (``gemma3.py:39-58``)."""
    if content_key.ndim != 3 or content_key.shape != value.shape:
        raise ValueError("Gemma K/V must have matching [tokens,heads,dim] shapes")
    tokens = content_key.shape[0]
    if prefix_length is not None and prefix_length != tokens:
        raise ValueError("prefix length must equal the materialized token count")
    first, _ = retained_window(tokens, layer_type=layer_type, sliding_window=sliding_window)
    return MaterializedKV(content_key[first:], value[first:], first, tokens)


def _gemma_roster_problems(cache, mapped, prefix_length: int) -> Iterator[Exception]:
    if set(mapped) != set(range(len(cache.layers))):
        yield ValueError("Gemma payload must cover every target layer")
        return
    for index, layer in enumerate(cache.layers):
        key, value = mapped[index]
        problem = _kv_pair_problem(key, value)
        if problem is not None:
            yield problem
        role = _role(layer)
        if role not in ("sliding", "full"):
            yield TypeError("Expected an attention cache layer")
        if getattr(layer, "is_initialized", False):
            yield ValueError(f"Target cache layer {index} is already initialized")
        # A sliding layer holds the last W - 1 tokens; its window is not re-validated here.
        expected = min(prefix_length, int(layer.sliding_window) - 1) if role == "sliding" else prefix_length
        if expected < 1 or key.shape[-2] != expected:
            yield ValueError(f"Invalid history length for layer {index}: expected {expected}")


def install_kv(cache, *, mapped, prefix_length):
    """Install RoPE-applied K/V into every layer of a native Gemma cache.

    ``mapped`` maps each layer index to ``(key, value)`` of shape
    ``[batch, heads, tokens, head_dim]``. The whole roster is checked first
    (coverage, geometry, layer kind, fresh layers, history length); only then
    is any layer updated, and a sliding layer records the whole prefix length
    as its cumulative length (``gemma3.py:61-94``).
    """
    _positive_int(prefix_length, "prefix_length")
    _raise_first(_gemma_roster_problems(cache, mapped, prefix_length))
    for index, layer in enumerate(cache.layers):
        layer.update(*mapped[index])
        if _role(layer) == "sliding":
            layer.cumulative_length = prefix_length


# ---------------------------------------------------------------------------
# Qwen3.5 (cb/architectures/qwen35.py)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class LinearLayerSpec:
    """The fields of a linear-attention ``LayerSpec`` (``cb/architectures/base.py:35-88``)
    that ``install_linear_state`` checks against."""

    index: int
    key_heads: int
    value_heads: int
    key_dim: int
    value_dim: int
    conv_kernel_size: int
    kind: str = "linear_attention"

    @property
    def conv_channels(self) -> int:
        return 2 * self.key_heads * self.key_dim + self.value_heads * self.value_dim


_DTYPES = {torch.float32: _lib.CB_DTYPE_F32, torch.float64: _lib.CB_DTYPE_F64}


def _batched(t: torch.Tensor, batch_shape: torch.Size) -> tuple[torch.Tensor, int]:
    """A contiguous operand for ``batch_shape`` and its batch stride in elements
    (0 when one matrix serves every batch entry)."""
    mat = t.shape[-2] * t.shape[-1]
    lead = t.shape[:-2]
    if lead == batch_shape:
        return t.contiguous(), mat
    if int(torch.Size(lead).numel()) == 1:
        return t.reshape(t.shape[-2], t.shape[-1]).contiguous(), 0
    return t.expand(*batch_shape, t.shape[-2], t.shape[-1]).contiguous(), mat


def transform_delta_state(source_state, key_basis, value_basis, *, stream=None):
    """Map recurrent memory as ``key_basis^T @ source_state @ value_basis``.

    ``source_state`` is ``[..., k, v]``, ``key_basis`` ``[..., k, k']`` and
    ``value_basis`` ``[..., v, v']``; leading dimensions broadcast as in the
    reference's matmul chain (``qwen35.py:52-61``). The result is
    ``[..., k', v']`` in the inputs' dtype (fp32 or fp64), computed on the GPU
    in one launch of ``cb_delta_state_transform``.
    """
    if min(source_state.ndim, key_basis.ndim, value_basis.ndim) < 2:
        raise ValueError("Delta state and basis tensors must be matrix-valued")
    if source_state.shape[-2] != key_basis.shape[-2] or source_state.shape[-1] != value_basis.shape[-2]:
        raise ValueError("Source state dimensions do not match the key/value bases")
    tensors = (source_state, key_basis, value_basis)
    if any(not t.is_cuda for t in tensors) or len({t.device for t in tensors}) != 1:
        raise ValueError("transform_delta_state needs its tensors on one GPU")
    if len({t.dtype for t in tensors}) != 1 or source_state.dtype not in _DTYPES:
        raise ValueError("Delta state and bases must share a dtype, float32 or float64")
    k, v = source_state.shape[-2:]
    kp, vp = key_basis.shape[-1], value_basis.shape[-1]
    batch_shape = torch.broadcast_shapes(source_state.shape[:-2], key_basis.shape[:-2], value_basis.shape[:-2])
    batch = int(batch_shape.numel())
    out = torch.empty(*batch_shape, kp, vp, dtype=source_state.dtype, device=source_state.device)
    if batch == 0:
        return out
    u, su = _batched(source_state, batch_shape)
    a, sa = _batched(key_basis, batch_shape)
    b, sb = _batched(value_basis, batch_shape)
    lib = _lib.load()
    with torch.cuda.device(source_state.device):
        _lib.check(lib.cb_delta_state_transform(
            _DTYPES[source_state.dtype], batch, k, v, kp, vp,
            u.data_ptr(), su, a.data_ptr(), sa, b.data_ptr(), sb,
            out.data_ptr(), kp * vp, _lib.stream_handle(stream)))
    return out


def required_replay(conv_kernel_size):
    """Suffix length that replaces zero convolution history (``qwen35.py:64-66``)."""
    return _positive_int(conv_kernel_size, "conv_kernel_size") - 1


def _attention_problems(cache, layer_index, key, value) -> Iterator[Exception]:
    if key.ndim != 4 or key.shape != value.shape or key.shape[-2] < 1:
        yield ValueError("K/V must match nonempty [batch,heads,tokens,head_dim]")
    if key.dtype != value.dtype or key.device != value.device:
        yield ValueError("K/V dtype and device must match")
    layer = cache.layers[layer_index]
    if _role(layer) != "full":
        yield TypeError("Expected a full-attention cache layer")
    if getattr(layer, "is_initialized", False):
        yield ValueError("Target cache layer is already initialized")


def install_attention_kv(cache, layer_index, key, value):
    """Install K/V into a fresh full-attention layer (``qwen35.py:69-82``)."""
    _raise_first(_attention_problems(cache, layer_index, key, value))
    cache.layers[layer_index].update(key, value)


def _linear_payload_problems(recurrent_state, conv_state, conv_kernel_size) -> Iterator[Exception]:
    if recurrent_state.ndim != 4 or conv_state.ndim != 3:
        yield ValueError("Expected recurrent [batch,heads,key,value] and convolution [batch,channels,kernel]")
        return
    _positive_int(conv_kernel_size, "conv_kernel_size")
    if conv_state.shape[-1] != conv_kernel_size or recurrent_state.shape[0] != conv_state.shape[0]:
        yield ValueError("Convolution length or batch geometry mismatch")
    if recurrent_state.device != conv_state.device:
        yield ValueError("Recurrent and convolution states must share a device")
    if not (recurrent_state.is_floating_point() and conv_state.is_floating_point()):
        yield ValueError("Recurrent and convolution states must be floating-point tensors")


def _linear_spec_problems(spec, layer_index, recurrent_state, conv_state,
                          conv_kernel_size) -> Iterator[Exception]:
    if spec.index != layer_index or spec.kind != "linear_attention":
        yield ValueError("Layer specification does not match the recurrent destination")
    if tuple(recurrent_state.shape[1:]) != (spec.value_heads, spec.key_dim, spec.value_dim):
        yield ValueError("Recurrent tensor does not match the layer specification")
    conv_shape = (spec.conv_channels, spec.conv_kernel_size)
    if tuple(conv_state.shape[1:]) != conv_shape or conv_kernel_size != spec.conv_kernel_size:
        yield ValueError("Convolution tensor does not match the layer specification")


def install_linear_state(cache, layer_index, *, recurrent_state, conv_state, conv_kernel_size, spec=None):
    """Install mapped recurrent memory and the receiver's convolution tail into a
    fresh linear-attention layer (``qwen35.py:85-160``). Every check runs
    before the layer is touched."""

    def problems():
        yield from _linear_payload_problems(recurrent_state, conv_state, conv_kernel_size)
        if spec is not None:
            yield from _linear_spec_problems(spec, layer_index, recurrent_state, conv_state, conv_kernel_size)
        layer = cache.layers[layer_index]
        if _role(layer) != "linear":
            yield TypeError("Target is not a linear-attention cache layer")
        elif bool(layer.has_previous_state[0]):
            yield ValueError("Target cache layer already has previous state")

    _raise_first(problems())
    layer = cache.layers[layer_index]
    layer.update_conv_state(conv_state, state_idx=0, conv_kernel_size=conv_kernel_size)
    layer.update_recurrent_state(recurrent_state, state_idx=0)
    if not bool(layer.has_previous_state[0]):
        raise RuntimeError("Linear cache did not enter previous-state mode")
