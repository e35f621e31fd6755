"""Slot runs and the byte geometry of run-segmented installs.

The reference installs a mapped block into unpublished pool pages run by run
(``_DirectMappedPoolCodec``, ``rt/source_mapper_adapter.py:366-428``, with
``rt/`` = ``src/cachebridge/backends/sglang/runtime/``): the token -> slot
vector is cut into maximal contiguous runs (``_contiguous_runs``, ``:349-363``)
and every (layer, run, kind) becomes one copy whose byte offsets
``operations`` (``cb/online/peer_geometry.py:4-54``) computes and checks.

On MI355X the fused kernel scatters rows straight through the slot vector or
block table, so runs are not needed to launch anything. These functions keep
the reference's geometry API (same arguments, tuples, order and ``ValueError``
messages) for callers that plan peer copies, and convert runs back to a slot
vector (``slots_from_runs``) for the kernel.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np
import torch

MAX_BLOCK_TOKENS = 4096


def contiguous_runs(values) -> list[tuple[int, int, int]]:
    """``(logical_start, logical_stop, physical_start)`` runs of a slot vector.

    A run ends wherever the next slot is not the previous slot plus one.
    """
    if isinstance(values, torch.Tensor):
        values = values.detach().cpu().numpy()
    v = np.asarray(list(values) if not isinstance(values, np.ndarray) else values, dtype=np.int64)
    if v.size == 0:
        return []
    cuts = np.flatnonzero(np.diff(v) != 1) + 1
    starts = np.concatenate(([0], cuts))
    stops = np.concatenate((cuts, [v.size]))
    return [(int(a), int(b), int(v[a])) for a, b in zip(starts, stops)]


def slots_from_runs(runs: Sequence[tuple[int, int, int]], start: int, stop: int,
                    device=None) -> torch.Tensor:
    """Slot of every token in ``[start, stop)`` from ordered runs (int64 tensor)."""
    out = np.empty(stop - start, dtype=np.int64)
    covered = 0
    for a, b, p in runs:
        lo, hi = max(start, a), min(stop, b)
        if lo < hi:
            out[lo - start: hi - start] = np.arange(p + lo - a, p + hi - a)
            covered += hi - lo
    if covered != stop - start:
        raise ValueError("target runs do not cover exactly one block")
    t = torch.from_numpy(out)
    return t.to(device) if device is not None else t


def operations(start, stop, runs, *, layers=64, heads=4, dim=128, itemsize=2):
    """Copy list ``(kind, layer, src_offset, dst_offset, bytes)`` of one block.

    The source is the mapped block ``[2, layers, n, heads, dim]`` (offsets from
    its start); destinations are byte offsets of the physical slot within a
    pool layer. Ordered layer-major, then run, then K before V. Rejects
    geometry other than the fixed 64-layer, head_dim 128, 2-byte pool with 2 or
    4 heads, blocks over 4096 tokens, runs that are not an ordered logical
    partition, physical runs that overlap, partial coverage of the block, and
    a copy total that differs from the block's size.
    """
    if (not 0 <= start < stop or stop - start > MAX_BLOCK_TOKENS
            or (layers, dim, itemsize) != (64, 128, 2) or heads not in (2, 4)):
        raise ValueError("unsupported fixed peer-copy geometry")
    n = stop - start
    row = heads * dim * itemsize
    cursor = 0
    spans = []
    covered = 0
    for run in runs:
        if len(run) != 3 or not all(isinstance(x, int) for x in run):
            raise ValueError("invalid ordered logical partition")
        a, b, p = run
        if a != cursor or b <= a or p < 0:
            raise ValueError("invalid ordered logical partition")
        cursor = b
        spans.append((p, p + b - a))
        covered += max(0, min(stop, b) - max(start, a))
    spans.sort()
    for (_, end), (begin, _) in zip(spans, spans[1:]):
        if end > begin:
            raise ValueError("target pages alias")
    if covered != n:
        raise ValueError("target runs do not cover exactly one block")
    clipped = [(max(start, a), min(stop, b), p + max(start, a) - a) for a, b, p in runs
               if max(start, a) < min(stop, b)]
    out = []
    for layer in range(layers):
        for lo, hi, phys in clipped:
            for kind in (0, 1):
                src = ((kind * layers + layer) * n + (lo - start)) * row
                out.append((kind, layer, src, phys * row, (hi - lo) * row))
    if sum(op[4] for op in out) != 2 * layers * n * row:
        raise ValueError("copy-byte invariant")
    return out
