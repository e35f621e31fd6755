"""Receiver-owned delivery of raw source rows, block by block, into two slots.

The reference's target side imports every source layer buffer and, for each
block, issues ``2 x 40 x runs`` peer copies of **all** 40 source layers into a
packed ``[2, 40, n, heads, 128]`` slot (``rt/native_cuda.py:28-131``,
``rt/native_channel.py:160-215``; slot ``(start // 2048) % 2``, reused only
after the map of its previous block has finished). ``SelectedBlockDelivery``
keeps that contract with two differences:

- only the source layers the mapper reads are moved (``mapper.source_layers``:
  16 of 40 at the configured TP4 share, so 2.5x fewer bytes);
- each block is one gather launch (``cb_copy_rows``) on the delivery stream,
  whatever the run structure of its slot indices. The kernel reads rows
  through per-layer pointers, which may be device-local or peer memory
  imported over xGMI (``hipIpcOpenMemHandle``); on one GPU they are local.

By default the delivery stream is the consumer's stream, so slot hand-over
needs no cross-stream event. A separate stream (``stream=``) works, with event
waits on both sides, but on one MI355X (ROCm 7.2) it is slower: a kernel
waiting on another stream's event starts 10-12 us after the kernel before it
on its own stream ends (about 1 us without the wait), and a gather running
beside the map slows both (TP4 share, 2048-token blocks: map 69 -> 96 us,
gather 20 -> 65 us), so 16 blocks take 1.76 ms instead of 1.47 ms.

The mapper then reads a slot through a per-layer pointer table in which every
delivered source layer points at its plane of the slot, so the plan and its
layer indices are unchanged. ``rt/`` is
``src/cachebridge/backends/sglang/runtime/`` of the reference.
"""

from __future__ import annotations

from typing import Sequence

import torch

from .. import _lib
from ..plan import Rows, copy_rows, rows_from_layers, rows_from_page
from ..pool import pool_rows


def _at_offset(rows: Rows, index_offset: int) -> Rows:
    """The same description with another index offset (no new device tables)."""
    c = _lib.CbRows.from_buffer_copy(rows.c)
    c.index_offset = index_offset
    return Rows(c, rows.dtype, rows.device, rows.keep)


def coalesced_runs(rows: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``(first_token, length)`` of every maximal run of consecutive physical
    rows in ``rows`` (a block's slot indices in token order), as int64 tensors.

    A span-by-span delivery (the reference's peer-copy path) issues one copy
    per run, kind and layer; ``SelectedBlockDelivery`` moves the block in one
    gather launch whatever the runs are.
    """
    r = rows.reshape(-1).to(torch.int64)
    n = r.numel()
    if n == 0:
        empty = torch.zeros(0, dtype=torch.int64, device=r.device)
        return empty, empty
    step = torch.ones(n, dtype=torch.bool, device=r.device)
    step[1:] = r[1:] != r[:-1] + 1  # a run starts where the row does not follow its predecessor
    first = torch.nonzero(step).flatten()
    ends = torch.cat([first[1:], torch.tensor([n], dtype=torch.int64, device=r.device)])
    return first, ends - first


class SelectedBlockDelivery:
    """Two receiver slots fed from a source pool's selected layers.

    ``indices`` are the request's source slots (int32 or int64, on the pool's
    device); block ``[start, stop)`` holds tokens ``indices[start:stop]``.
    ``layers`` are global source layer ids (e.g. ``mapper.source_layers``).
    ``head_offset`` is the global index of the pool's first KV head (the
    rank's ``source_head_offset``).
    """

    def __init__(self, source_pool, indices: torch.Tensor, *, layers: Sequence[int], block_tokens: int,
                 head_offset: int = 0, stream: torch.cuda.Stream | None = None, slots: int = 2):
        first = source_pool._get_key_buffer(source_pool.start_layer)
        self.pool = source_pool
        self.pool_rows, self.heads, self.dim = first.shape
        self.dtype, self.device = first.dtype, first.device
        self.layers = tuple(sorted(set(int(l) for l in layers)))
        if not self.layers or self.layers[0] < 0 or self.layers[-1] >= source_pool.layer_num:
            raise ValueError("delivered layers must be source pool layers")
        if block_tokens < 1:
            raise ValueError("block_tokens must be positive")
        if indices.ndim != 1 or indices.dtype not in (torch.int32, torch.int64) or indices.device != self.device:
            raise ValueError("one-dimensional integer slot indices on the pool's device required")
        self.indices = indices
        self.block_tokens = int(block_tokens)
        self.head_offset = int(head_offset)
        self.stream = stream if stream is not None else torch.cuda.current_stream(self.device)
        n_sel = len(self.layers)
        self._storage = [torch.empty(2 * n_sel * self.block_tokens * self.heads * self.dim, dtype=self.dtype,
                                     device=self.device) for _ in range(slots)]
        self._ready = [torch.cuda.Event() for _ in range(slots)]
        self._free = [torch.cuda.Event() for _ in range(slots)]
        self._busy = [False] * slots
        self._released_on = [None] * slots  # stream of each slot's last consumer
        self._block = [None] * slots
        # Descriptions (and their device pointer tables) are built once and
        # live as long as this object: the kernels that read them run
        # asynchronously, and rebuilding them per block costs more host time
        # than a block's map.
        self._tables: dict = {}
        self._rows: dict = {}
        ks = [source_pool._get_key_buffer(source_pool.start_layer + l) for l in self.layers]
        vs = [source_pool._get_value_buffer(source_pool.start_layer + l) for l in self.layers]
        with torch.cuda.stream(self.stream):
            self._source = rows_from_layers(ks, vs, index=indices, tokens=len(indices),
                                            pointer_cache=self._tables.setdefault("source", {}))
        self.launches = 0
        self.logical_bytes = 0

    @property
    def slot_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self._storage)

    def span_copies(self, start: int, stop: int) -> int:
        """Copies a span-by-span delivery of block ``[start, stop)`` would issue
        (one per run of consecutive rows, kind and delivered layer); this
        class issues one launch."""
        first, _ = coalesced_runs(self.indices[start:stop])
        return 2 * len(self.layers) * int(first.numel())

    def deliver(self, slot: int, start: int, stop: int) -> torch.Tensor:
        """Gather block ``[start, stop)`` into ``slot`` on the delivery stream.

        Waits (on the device) for the slot's previous consumer; returns the
        packed ``[2, layers, n, heads, dim]`` view of the slot.
        """
        n = stop - start
        if not 0 <= start < stop <= len(self.indices) or n > self.block_tokens:
            raise ValueError("invalid block span")
        if self._block[slot] is not None:
            raise RuntimeError("slot still holds an unconsumed block")
        view = self._storage[slot][: 2 * len(self.layers) * n * self.heads * self.dim].view(
            2, len(self.layers), n, self.heads, self.dim)
        key = ("slot", slot, n)
        if key not in self._rows:
            self._rows[key] = rows_from_page(view)
        with torch.cuda.stream(self.stream):
            if self._busy[slot] and self._released_on[slot] != self.stream:
                self.stream.wait_event(self._free[slot])
            copy_rows(_at_offset(self._source, start), self._rows[key], num_layers=len(self.layers),
                      num_tokens=n, row_elements=int(self.heads * self.dim), stream=self.stream)
            self._ready[slot].record(self.stream)
        self._busy[slot] = True
        self._block[slot] = (start, stop, view)
        self.launches += 1
        self.logical_bytes += 2 * len(self.layers) * n * self.heads * self.dim * self.dtype.itemsize
        return view

    def source_rows(self, slot: int, stream: torch.cuda.Stream) -> Rows:
        """Source description of the slot's block for ``mapper.map_install`` on
        ``stream``: layer ``l`` of the source model reads plane
        ``layers.index(l)`` (other layers are never read and alias plane 0)."""
        if self._block[slot] is None:
            raise RuntimeError("slot holds no delivered block")
        _, _, view = self._block[slot]
        key = ("planes", slot, view.shape[2])
        if key not in self._rows:
            plane = {l: i for i, l in enumerate(self.layers)}
            depth = self.layers[-1] + 1
            ks = [view[0, plane.get(l, 0)] for l in range(depth)]
            vs = [view[1, plane.get(l, 0)] for l in range(depth)]
            with torch.cuda.stream(stream):  # the pointer table is uploaded ahead of the map
                self._rows[key] = rows_from_layers(ks, vs, head_offset=self.head_offset,
                                                   pointer_cache=self._tables.setdefault(key, {}))
        return self._rows[key]

    def consume(self, slot: int, stream: torch.cuda.Stream) -> tuple[int, int]:
        """Make ``stream`` wait for the slot's delivery; returns the block span."""
        if self._block[slot] is None:
            raise RuntimeError("slot holds no delivered block")
        if stream != self.stream:
            stream.wait_event(self._ready[slot])
        start, stop, _ = self._block[slot]
        return start, stop

    def release(self, slot: int, stream: torch.cuda.Stream) -> None:
        """The slot's reads are enqueued on ``stream``; the next delivery into
        the slot waits for them on the device."""
        if self._block[slot] is None:
            raise RuntimeError("slot holds no delivered block")
        if stream != self.stream:
            self._free[slot].record(stream)
        self._released_on[slot] = stream
        self._block[slot] = None

    def receipt(self) -> dict:
        return dict(input_copy="one gather launch per block (cb_copy_rows)", launches=self.launches,
                    logical_input_bytes=self.logical_bytes, delivered_layers=list(self.layers),
                    slot_bytes=self.slot_bytes)


@torch.inference_mode()
def map_install_delivered(mapper, delivery: SelectedBlockDelivery, slot: int, target_pool, *,
                          target_indices=None, block_table=None, page_size=None, prefix_length=0,
                          stream: torch.cuda.Stream | None = None) -> tuple[int, int]:
    """Map the block delivered into ``slot`` and install it into the target pool.

    Runs on ``stream`` (default: the current stream) after the slot's delivery,
    then releases the slot. Tokens sit at positions ``start + t``; target rows
    come from ``target_indices[start:stop]`` or from ``block_table`` with
    ``page_size``, as in ``map_install_block``.
    """
    s = stream if stream is not None else torch.cuda.current_stream()
    start, stop = delivery.consume(slot, s)
    n = stop - start
    if (target_indices is None) == (block_table is None):
        raise ValueError("give exactly one of target_indices or block_table")
    if block_table is not None:
        ps = page_size if page_size is not None else getattr(target_pool, "page_size", None)
        target = pool_rows(target_pool, block_table=block_table, page_size=ps, index_offset=start, tokens=n)
    else:
        if stop > len(target_indices):
            raise ValueError("invalid target range")
        target = pool_rows(target_pool, index=target_indices, index_offset=start, tokens=n)
    mapper.map_install(delivery.source_rows(slot, s), target, num_tokens=n, position_start=start,
                       prefix_length=prefix_length, stream=s)
    delivery.release(slot, s)
    return start, stop
