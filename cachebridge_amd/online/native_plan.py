"""Receiver-side delivery geometry of raw source rows for one block.

``build_plan`` mirrors ``rt/native_plan.py:1-95`` (``rt/`` =
``src/cachebridge/backends/sglang/runtime/`` of the reference): the block's
physical source rows ``indices[start:stop]`` are coalesced into runs of
consecutive rows, keeping logical token order, and ``Plan.spans()`` lists the
per-(kind, layer, run) byte copies into a packed ``[2, layers, n, heads, dim]``
block. The reference executes those spans as ``2 x layers x runs`` peer copies
(``rt/native_cuda.py:108-131``); ``cachebridge_amd.online.delivery`` moves the
same rows with one gather launch and, with ``layers`` restricted to the
source layers the mapper reads, ships only those.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Run:
    source_row: int
    destination_token: int
    rows: int


@dataclass(frozen=True)
class Plan:
    start: int
    stop: int
    pool_rows: int
    layers: int
    heads: int
    dimension: int
    element_bytes: int
    runs: tuple

    @property
    def useful_bytes(self) -> int:
        return 2 * self.layers * (self.stop - self.start) * self.heads * self.dimension * self.element_bytes

    @property
    def copy_calls(self) -> int:
        """Copies the span-by-span execution issues (one per kind, layer and run)."""
        return 2 * self.layers * len(self.runs)

    def spans(self):
        """Per-(kind, layer, run) copies: byte offset in the source layer, byte
        offset in the packed block, length."""
        n = self.stop - self.start
        row_bytes = self.heads * self.dimension * self.element_bytes
        for kind in range(2):
            for layer in range(self.layers):
                for run in self.runs:
                    yield dict(kind=kind, layer=layer,
                               source_byte_offset=run.source_row * row_bytes,
                               destination_byte_offset=((kind * self.layers + layer) * n
                                                        + run.destination_token) * row_bytes,
                               bytes=run.rows * row_bytes)


def build_plan(indices, *, start, stop, pool_rows, layers=40, heads=2, dimension=128, element_bytes=2) -> Plan:
    """Coalesce adjacent physical rows of ``indices[start:stop]`` into runs."""
    geometry = (start, stop, pool_rows, layers, heads, dimension, element_bytes)
    if any(type(x) is not int for x in geometry):
        raise ValueError("integer geometry required")
    if (not 0 <= start < stop <= len(indices) or min(pool_rows, layers, heads, dimension, element_bytes) <= 0
            or element_bytes != 2):
        raise ValueError("invalid geometry")
    rows = tuple(indices[start:stop])
    if any(type(row) is not int or not 0 <= row < pool_rows for row in rows):
        raise ValueError("native row outside certified pool geometry")
    runs = []
    i = 0
    while i < len(rows):
        j = i + 1
        while j < len(rows) and rows[j] == rows[j - 1] + 1:
            j += 1
        runs.append(Run(rows[i], i, j - i))
        i = j
    return Plan(start, stop, pool_rows, layers, heads, dimension, element_bytes, tuple(runs))
