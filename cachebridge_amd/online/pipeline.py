"""Double-buffered handoff: the two-slot source lease and the two-stream staged install.

- ``PipelinedSourceLease``: ``cb/online/pipeline.py:7-43`` (=
  ``rt/source_mapper_adapter.py:91-127``): one source lock held while at most
  one export per output slot is live; a slot is reused only after its
  consumer reports GPU completion.
- ``StagedHandoff``: the reference's bounded, double-buffered block loop
  (``rt/source_mapper_adapter.py:597-831``: map into output slot
  ``blocks % 2`` on a compute stream, record an event, install on another
  stream, reuse a slot only after its install completed) restated over target
  **layer chunks**: chunk ``i+1`` is reconstructed into staging slot
  ``(i+1) % 2`` on ``compute_stream`` while chunk ``i`` is scattered from
  its slot into the target pool on ``install_stream``. Temporary memory is
  ``2 x [2, layer_chunk, max_tokens, heads, head_dim]``.

``rt/`` is ``src/cachebridge/backends/sglang/runtime/`` of the reference.

When the target pool is directly addressable by the device (the common case),
``HeadwiseMapper.map_install`` writes it in one fused launch with no staging at
all; the staged path is for installs that must go through a separate copy
(a pool whose rows the map kernel must not write until a slot is ready, or a
copy engine / peer link on the install side).
"""

from __future__ import annotations

from typing import Sequence

import torch

from ..layouts import FULL, SLIDING, retained_window
from ..plan import Rows, copy_rows, rows_from_layers, rows_from_page


class PipelinedSourceLease:
    """One source lock; at most one live export per output slot."""

    def __init__(self, acquire, release, slots: int = 2):
        self.acquire = acquire
        self.release = release
        self.pending = [False] * slots
        self.active = False
        self.next_start = 0

    def begin(self):
        if self.active:
            raise RuntimeError("pipelined source lease already active")
        self.acquire()
        self.active = True

    def export(self, slot, start, stop):
        ordered = start == self.next_start and stop > start
        if not self.active or self.pending[slot] or not ordered:
            raise RuntimeError("pipelined block ownership/order violation")
        self.pending[slot] = True
        self.next_start = stop

    def acknowledge(self, slot, *, gpu_reads_complete):
        if not (self.active and self.pending[slot] and gpu_reads_complete):
            raise RuntimeError("slot-local GPU completion required before reuse")
        self.pending[slot] = False

    def close(self):
        if not self.active or any(self.pending):
            raise RuntimeError("cannot release source lease with live output slots")
        self.release()
        self.active = False


def layer_chunks(windows: Sequence, layer_chunk: int) -> list[list[int]]:
    """Target layers grouped by window class (full first), ``layer_chunk`` at most each."""
    if layer_chunk < 1:
        raise ValueError("layer_chunk must be positive")
    order = sorted(range(len(windows)), key=lambda l: (windows[l] is not None, windows[l] or 0, l))
    chunks: list[list[int]] = []
    for l in order:
        if chunks and len(chunks[-1]) < layer_chunk and windows[chunks[-1][0]] == windows[l]:
            chunks[-1].append(l)
        else:
            chunks.append([l])
    return chunks


class StagedHandoff:
    """Two-stream layer-chunk pipeline over one ``HeadwiseMapper``.

    ``run`` is asynchronous: it orders its work after the caller's current
    stream and makes the current stream wait for the last install, so work the
    caller enqueues afterwards (publication, frees) sees the installed pool.
    """

    def __init__(self, mapper, *, layer_chunk: int = 4, max_tokens: int = 4096,
                 compute_stream: torch.cuda.Stream | None = None,
                 install_stream: torch.cuda.Stream | None = None):
        self.mapper = mapper
        self.device = mapper.device
        self.max_tokens = int(max_tokens)
        if self.max_tokens < 1:
            raise ValueError("max_tokens must be positive")
        self.chunks = layer_chunks(mapper.windows, layer_chunk)
        self.plans = [mapper.layer_plan(c) for c in self.chunks]
        width = max(len(c) for c in self.chunks)
        self.staging = torch.empty(2, 2, width, self.max_tokens, mapper.local_heads,
                                   mapper.head_dim, dtype=mapper.dtype, device=self.device)
        self.compute_stream = compute_stream or torch.cuda.Stream(device=self.device)
        self.install_stream = install_stream or torch.cuda.Stream(device=self.device)
        self._mapped = [torch.cuda.Event() for _ in range(2)]
        self._installed = [torch.cuda.Event() for _ in range(2)]
        self._pointer_caches = [dict() for _ in self.chunks]

    @property
    def staging_bytes(self) -> int:
        return self.staging.numel() * self.staging.element_size()

    def _first_kept(self, layer: int, position_start: int, tokens: int, prefix: int) -> int:
        window = self.mapper.windows[layer]
        kind = FULL if window is None else SLIDING
        first, _ = retained_window(prefix, layer_type=kind, sliding_window=window)
        return min(tokens, max(0, first - position_start))

    def run(self, source: Rows, target_pool, *, num_tokens: int, position_start: int,
            index: torch.Tensor | None = None, block_table: torch.Tensor | None = None,
            page_size: int | None = None, index_offset: int = 0, prefix_length: int = 0) -> None:
        """Map + install one block of ``num_tokens`` tokens through the staging slots.

        ``target_pool`` is an SGLang-style pool (``start_layer``,
        ``_get_key_buffer``, ``_get_value_buffer``); ``index`` (token -> slot)
        or ``block_table`` + ``page_size`` place token ``t`` at
        ``index_offset + t`` of the request's slot space.
        """
        n = int(num_tokens)
        if not 0 < n <= self.max_tokens:
            raise ValueError(f"block of {n} tokens does not fit {self.max_tokens}-token staging")
        self.mapper._check_positions(position_start, n)
        prefix = int(prefix_length) if prefix_length > 0 else position_start + n
        if prefix < position_start + n:
            raise ValueError("prefix_length is shorter than the block end")
        heads, dim = self.mapper.local_heads, self.mapper.head_dim
        start = target_pool.start_layer
        # Descriptors first: their device pointer arrays are uploaded on the
        # current stream, which both pipeline streams wait for below.
        steps = []
        for i, layers in enumerate(self.chunks):
            keep = self._first_kept(layers[0], position_start, n, prefix)
            staged = rows_from_page(self.staging[i % 2])
            staged.c.num_layers = len(layers)
            dst = None
            if keep < n:
                dst = rows_from_layers(
                    [target_pool._get_key_buffer(start + l) for l in layers],
                    [target_pool._get_value_buffer(start + l) for l in layers],
                    index=index, block_table=block_table, page_size=page_size,
                    index_offset=index_offset + keep, tokens=n - keep,
                    pointer_cache=self._pointer_caches[i])
            steps.append((staged, dst, keep))
        current = torch.cuda.current_stream(self.device)
        cs, ins = self.compute_stream, self.install_stream
        cs.wait_stream(current)
        ins.wait_stream(current)
        for i, (plan, (staged, dst, keep)) in enumerate(zip(self.plans, steps)):
            slot = i % 2
            if i >= 2:
                cs.wait_event(self._installed[slot])
            plan.launch(source, staged, num_tokens=n, position_start=position_start,
                        prefix_length=prefix, stream=cs)
            self._mapped[slot].record(cs)
            ins.wait_event(self._mapped[slot])
            if dst is not None:
                src = rows_from_page(self.staging[slot])
                src.c.index_offset = keep
                copy_rows(src, dst, num_layers=staged.c.num_layers, num_tokens=n - keep,
                          row_elements=heads * dim, stream=ins)
            self._installed[slot].record(ins)
        current.wait_stream(cs)
        current.wait_stream(ins)
