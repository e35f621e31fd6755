"""Block packing, fused map+install and the unpublished-install transaction.

Same names, argument meaning and error behaviour as the reference primitives
(``cb/online/blocks.py:11-171``); the data movement runs in
``libcachebridge_hip`` on the caller's current stream.

- ``SourceLease``: single in-flight block lease (``cb/online/blocks.py:11-43``).
- ``pack_source_block``: gather pool rows into a contiguous workspace
  (``cb/online/blocks.py:47-82``) with one row-copy launch for all layers.
- ``map_write_block``: map a packed block and write it into the target pool
  rows (``cb/online/blocks.py:86-111``) in one fused launch, without the
  intermediate mapped tensor.
- ``map_install_block``: gather + map + install straight from the source pool
  (no packed block at all), through a token-slot vector or a block table.
- ``map_install_batch``: the same for a ragged batch of requests (an admitted
  cohort, ``cb/online/admission.py:420-499``) in one launch.
- ``install_unpublished``: allocate, write all blocks in order, vote, then
  publish or roll back (``cb/online/blocks.py:114-171``).
"""

from __future__ import annotations

import torch

from ..plan import RequestSpan, copy_rows, rows_from_page
from ..pool import pool_rows


class SourceLease:
    """Single in-flight block; release is legal only after consumer completion."""

    def __init__(self, acquire, release):
        self.acquire = acquire
        self.release = release
        self.active = False
        self.pending = False
        self.next_start = 0

    def begin(self):
        if self.active:
            raise RuntimeError("source lease already active")
        self.acquire()
        self.active = True
        self.next_start = 0

    def export(self, start, stop):
        if not self.active or self.pending or start != self.next_start or stop <= start:
            raise RuntimeError("block ownership/order violation")
        self.pending = True
        self.next_start = stop

    def acknowledge(self, *, gpu_reads_complete):
        if not self.active or not self.pending or not gpu_reads_complete:
            raise RuntimeError("consumer GPU completion required before buffer reuse")
        self.pending = False

    def close(self):
        if not self.active or self.pending:
            raise RuntimeError("cannot release source lease with outstanding GPU reads")
        self.release()
        self.active = False


def _pool_geometry(pool):
    first = pool._get_key_buffer(pool.start_layer)
    return first, first.shape[1], first.shape[2]


@torch.inference_mode()
def pack_source_block(pool, indices, *, start, stop, workspace, block_tokens):
    """Gather ``indices[start:stop]`` rows of every pool layer into ``workspace``.

    Returns the ``[2, layers, n, heads, head_dim]`` view of the workspace prefix.
    """
    n = stop - start
    if not 0 <= start < stop <= len(indices) or n > block_tokens:
        raise ValueError("invalid block span")
    layers = pool.layer_num
    first, heads, dim = _pool_geometry(pool)
    required = 2 * layers * block_tokens * heads * dim
    if workspace.ndim != 1 or workspace.numel() != required or not workspace.is_contiguous():
        raise ValueError("workspace must be exactly one contiguous block")
    if (workspace.device != first.device or workspace.dtype != first.dtype
            or indices.device != first.device):
        raise ValueError("pool, indices and workspace must share device and dtype as applicable")
    if indices.ndim != 1 or indices.dtype not in (torch.int32, torch.int64):
        raise ValueError("one-dimensional integer pool indices required")
    block = workspace[: 2 * layers * n * heads * dim].view(2, layers, n, heads, dim)
    src = pool_rows(pool, index=indices, index_offset=start, tokens=n)
    copy_rows(src, rows_from_page(block), num_layers=layers, num_tokens=n,
              row_elements=heads * dim)
    return block


@torch.inference_mode()
def map_write_block(mapper, block, target_pool, target_indices, *, start, source_head_offset):
    """Map a packed ``[2, Ls, n, Hs, D]`` block into ``target_indices[start:start+n]`` rows."""
    n = block.shape[2]
    if start < 0 or start + n > len(target_indices) or mapper.method != "cachebridge":
        raise ValueError("invalid target range or non-CacheBridge method")
    first, heads, dim = _pool_geometry(target_pool)
    if (target_pool.layer_num != mapper.target_layers or target_pool.dtype != block.dtype
            or heads != mapper.local_heads or dim != block.shape[4]):
        raise ValueError("mapper output geometry/dtype mismatch")
    if block.device != first.device:
        raise ValueError("block and target pool must share a device")
    page = block if block.is_contiguous() else block.contiguous()
    source = rows_from_page(page, head_offset=source_head_offset)
    target = pool_rows(target_pool, index=target_indices.to(first.device), index_offset=start,
                       tokens=n)
    mapper.map_install(source, target, num_tokens=n, position_start=start)


@torch.inference_mode()
def map_install_block(mapper, source_pool, source_indices, target_pool, *, start, stop,
                      target_indices=None, block_table=None, page_size=None,
                      source_head_offset=0, prefix_length=0, stream=None,
                      tokens_per_workgroup=0):
    """Gather ``source_indices[start:stop]`` rows, map them and install them.

    Target rows come from ``target_indices[start:stop]`` (token slots, the
    reference's page_size=1 layout) or from ``block_table`` with ``page_size``
    (token ``u`` of the request lives at ``bt[u // ps] * ps + u % ps``).
    Tokens sit at positions ``start + t``. Asynchronous on ``stream``.
    """
    n = stop - start
    if not 0 <= start < stop <= len(source_indices):
        raise ValueError("invalid block span")
    if (target_indices is None) == (block_table is None):
        raise ValueError("give exactly one of target_indices or block_table")
    if target_pool.layer_num != mapper.target_layers:
        raise ValueError("mapper output geometry/dtype mismatch")
    source = pool_rows(source_pool, index=source_indices, index_offset=start, tokens=n,
                       head_offset=source_head_offset)
    if block_table is not None:
        ps = page_size if page_size is not None else getattr(target_pool, "page_size", None)
        target = pool_rows(target_pool, block_table=block_table, page_size=ps, index_offset=start,
                           tokens=n)
    else:
        if start + n > len(target_indices):
            raise ValueError("invalid target range")
        target = pool_rows(target_pool, index=target_indices, index_offset=start, tokens=n)
    mapper.map_install(source, target, num_tokens=n, position_start=start,
                       prefix_length=prefix_length, stream=stream,
                       tokens_per_workgroup=tokens_per_workgroup)


def map_install_batch(mapper, source_pool, source_indices, target_pool, requests, *,
                      target_indices=None, block_table=None, page_size=None,
                      source_head_offset=0, stream=None):
    """Gather, map and install every request of a ragged batch in one launch.

    ``requests`` are ``RequestSpan(source_offset, target_offset, num_tokens,
    position_start, prefix_length)``: request token ``t`` reads source row
    ``source_indices[source_offset + t]`` and writes target row
    ``target_indices[target_offset + t]``, or, with ``block_table``, target
    row ``bt[u // ps] * ps + u % ps`` at ``u = target_offset + t`` (so a
    request whose pages start at block-table entry ``e`` has
    ``target_offset = e * ps``). Every row equals what ``map_install_block``
    writes for that request alone. Asynchronous on ``stream``.
    """
    spans = [RequestSpan(*r) for r in requests]
    if (target_indices is None) == (block_table is None):
        raise ValueError("give exactly one of target_indices or block_table")
    if target_pool.layer_num != mapper.target_layers:
        raise ValueError("mapper output geometry/dtype mismatch")
    for sp in spans:
        if sp.num_tokens < 0 or sp.source_offset < 0 or sp.target_offset < 0:
            raise ValueError("invalid request span")
    src_end = max((sp.source_offset + sp.num_tokens for sp in spans if sp.num_tokens), default=0)
    tgt_end = max((sp.target_offset + sp.num_tokens for sp in spans if sp.num_tokens), default=0)
    if src_end > len(source_indices):
        raise ValueError("a request reads past the end of source_indices")
    source = pool_rows(source_pool, index=source_indices, head_offset=source_head_offset)
    if block_table is not None:
        ps = page_size if page_size is not None else getattr(target_pool, "page_size", None)
        target = pool_rows(target_pool, block_table=block_table, page_size=ps, tokens=tgt_end)
    else:
        if tgt_end > len(target_indices):
            raise ValueError("a request writes past the end of target_indices")
        target = pool_rows(target_pool, index=target_indices)
    mapper.map_install_batch(source, target, spans, stream=stream)


def install_unpublished(*, token_count, allocate, free, blocks, write, synchronize, ready_vote,
                        publish, cancel_after_blocks=None):
    """Unpublished target transaction (``cb/online/blocks.py:114-171`` semantics).

    ``blocks`` yields ``(start, stop, value)`` in order; ``value`` is the
    block's mapped page ``[2, layers, n, heads, D]`` (the reference's
    ``map_write_block`` flow) or, for the fused install, the block's 1-D
    source-row slice (``n`` entries). ``write(value, indices, start)`` enqueues
    the install; ``synchronize()`` fences it. No page is published while any
    rank may still be writing: ``ready_vote`` runs on every rank even after a
    local failure; a failed or cancelled transaction frees its pages exactly
    once; a broken vote keeps them owned.
    """
    indices = None
    error = None
    count = 0
    cursor = 0
    try:
        indices = allocate(token_count)
        if indices is None:
            raise RuntimeError("target pool allocation failed")
        for start, stop, value in blocks:
            tokens = value.shape[2] if value.ndim >= 3 else value.shape[0]
            if start != cursor or not start < stop <= token_count or tokens != stop - start:
                raise ValueError("missing, duplicate or overlapping block")
            write(value, indices, start)
            synchronize()
            cursor = stop
            count += 1
            if cancel_after_blocks == count:
                raise RuntimeError("controlled cancellation before publication")
        if cursor != token_count:
            raise ValueError("incomplete prefix")
    except Exception as exc:  # noqa: BLE001 -- every local failure must reach the vote
        error = exc
    synchronize()
    all_ready = ready_vote(error is None)
    if error is not None or not all_ready:
        if indices is not None:
            free(indices)
        raise RuntimeError("unpublished target transaction rolled back") from error
    publish(indices)
    return dict(tokens=cursor, blocks=count, published=True)
