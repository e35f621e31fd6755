"""Target-layout rules the handoff plan needs: head ownership and attention windows.

- ``head_assignment``: ``cb/architectures/base.py:116-135`` (identity for equal
  KV-head counts, an explicit per-target-head source head otherwise).
- ``gemma_layer_types``: the implicit Gemma 3 local/global pattern
  (``cb/architectures/gemma3.py:12-28``): layer ``i`` is full attention when
  ``(i + 1) % pattern == 0``, sliding otherwise.
- ``retained_window``: ``cb/architectures/gemma3.py:39-58``: a sliding layer
  keeps the last ``min(prefix, W - 1)`` tokens of the prefix, a full layer all
  of them. The fused kernel applies the same rule per window class; this
  function is its host statement (plan set-up and validation).
- ``mapper_windows``: per-target-layer ``windows`` argument of
  ``HeadwiseMapper`` from layer types.
"""

from __future__ import annotations

from typing import Sequence

SLIDING = "sliding_attention"
FULL = "full_attention"


def _positive_int(value, name: str) -> int:
    if type(value) is not int or value < 1:
        raise ValueError(f"{name} must be a positive integer")
    return value


def head_assignment(source_heads, target_heads, assignment: Sequence[int] | None = None):
    """Source KV head of every target KV head (a tuple of length ``target_heads``)."""
    _positive_int(source_heads, "source_heads")
    _positive_int(target_heads, "target_heads")
    if assignment is None:
        if source_heads != target_heads:
            raise ValueError("Unequal KV-head counts require an explicit head assignment")
        return tuple(range(target_heads))
    heads = tuple(assignment)
    if len(heads) != target_heads or any(type(h) is not int or not 0 <= h < source_heads
                                         for h in heads):
        raise ValueError("Head assignment must identify a valid source head for each target head")
    return heads


def gemma_layer_types(num_layers: int, pattern: int = 6) -> list[str]:
    """Implicit Gemma 3 layer kinds: every ``pattern``-th layer is full attention."""
    _positive_int(num_layers, "num_hidden_layers")
    _positive_int(pattern, "sliding_window_pattern")
    return [FULL if (i + 1) % pattern == 0 else SLIDING for i in range(num_layers)]


def retained_window(prefix_length: int, *, layer_type: str, sliding_window=None) -> tuple[int, int]:
    """``(first_position, retained_tokens)`` of a layer for a ``prefix_length`` history."""
    if type(prefix_length) is not int or prefix_length < 1:
        raise ValueError("prefix length must equal the materialized token count")
    if layer_type == SLIDING:
        if _positive_int(sliding_window, "sliding_window") < 2:
            raise ValueError("Sliding window must leave room for the next token")
        retained = min(prefix_length, sliding_window - 1)
    elif layer_type == FULL:
        retained = prefix_length
    else:
        raise ValueError(f"Unsupported Gemma layer type: {layer_type}")
    return prefix_length - retained, retained


def mapper_windows(layer_types: Sequence[str], sliding_window: int) -> list[int | None]:
    """``windows`` for ``HeadwiseMapper``: the window size on sliding layers, else None."""
    out: list[int | None] = []
    for kind in layer_types:
        if kind == SLIDING:
            if _positive_int(sliding_window, "sliding_window") < 2:
                raise ValueError("Sliding window must leave room for the next token")
            out.append(int(sliding_window))
        elif kind == FULL:
            out.append(None)
        else:
            raise ValueError(f"Unsupported Gemma layer type: {kind}")
    return out
