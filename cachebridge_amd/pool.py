"""Paged KV pool on one GPU with SGLang's ``MHATokenToKVPool`` duck type.

The handoff path consumes a pool through ``layer_num``, ``start_layer``,
``dtype``, ``_get_key_buffer(layer)``, ``_get_value_buffer(layer)`` and
``set_kv_buffer(layer, loc, k, v, layer_id_override=...)``
(``cb/online/blocks.py:57-59,79-81,106-111``). ``PagedKVPool`` provides that
surface over one ``[layers, rows, heads, head_dim]`` allocation per K and V
(per-layer views, so both per-layer pointer arrays and the stacked stride
describe it), with rows grouped in pages of ``page_size`` slots. ``pool_rows``
describes any object with that duck type (e.g. a real SGLang pool) for the
HIP kernels.
"""

from __future__ import annotations

import weakref

import torch

from .plan import Rows, copy_rows, rows_from_layers, rows_from_page, rows_from_stacked


class PagedKVPool:
    def __init__(self, *, layer_num: int, pages: int, head_num: int, head_dim: int,
                 page_size: int = 16, dtype: torch.dtype = torch.bfloat16, device="cuda",
                 start_layer: int = 0, fill: str | None = None):
        if page_size < 1 or pages < 1:
            raise ValueError("pages and page_size must be positive")
        self.layer_num = int(layer_num)
        self.start_layer = int(start_layer)
        self.page_size = int(page_size)
        self.pages = int(pages)
        self.size = self.pages * self.page_size
        self.head_num = int(head_num)
        self.head_dim = int(head_dim)
        self.dtype = dtype
        self.device = torch.device(device)
        shape = (self.layer_num, self.size, self.head_num, self.head_dim)
        self.k_data = torch.empty(shape, dtype=dtype, device=self.device)
        self.v_data = torch.empty(shape, dtype=dtype, device=self.device)
        if fill == "zeros":
            self.k_data.zero_()
            self.v_data.zero_()
        self.k_buffer = list(self.k_data.unbind(0))
        self.v_buffer = list(self.v_data.unbind(0))

    def _get_key_buffer(self, layer: int) -> torch.Tensor:
        return self.k_buffer[layer - self.start_layer]

    def _get_value_buffer(self, layer: int) -> torch.Tensor:
        return self.v_buffer[layer - self.start_layer]

    def rows(self, *, index=None, block_table=None, page_size=None, index_offset: int = 0,
             head_offset: int = 0, tokens=None, layers: slice | None = None) -> Rows:
        """Describe this pool (optionally a layer sub-range) with a token -> row index.

        K and V are each one ``[layers, rows, heads, head_dim]`` tensor, so the
        description is a base address and a layer stride: no per-layer pointer
        table and no per-layer checks on every call.
        """
        k, v = self.k_data, self.v_data
        if layers is not None:
            k, v = k[layers], v[layers]
        if block_table is not None and page_size is None:
            page_size = self.page_size
        return rows_from_stacked(k, v, index=index, block_table=block_table, page_size=page_size,
                                 index_offset=index_offset, head_offset=head_offset, tokens=tokens)

    def set_kv_buffer(self, layer, loc, cache_k, cache_v, k_scale=None, v_scale=None,
                      layer_id_override=None):
        """Row store ``buffer[layer][loc] = k`` on the GPU (SGLang semantics, no scale)."""
        index = layer_id_override if layer_id_override is not None else layer.layer_id
        if k_scale is not None or v_scale is not None:
            raise ValueError("scaled KV stores are not supported")
        if cache_k.dtype != self.dtype:
            cache_k = cache_k.to(self.dtype)
            cache_v = cache_v.to(self.dtype)
        n = int(loc.numel())
        if n == 0:
            return
        page = torch.stack((cache_k.reshape(n, self.head_num, self.head_dim),
                            cache_v.reshape(n, self.head_num, self.head_dim)))[:, None].contiguous()
        li = index - self.start_layer
        dst = self.rows(index=loc.to(self.device).contiguous(), layers=slice(li, li + 1), tokens=n)
        copy_rows(rows_from_page(page), dst, num_layers=1, num_tokens=n,
                  row_elements=self.head_num * self.head_dim)


# Per-pool device tables of per-layer K/V pointers, for pools that are not a
# PagedKVPool (one buffer per layer, e.g. SGLang's MHATokenToKVPool): built
# once per pool and rebuilt only when the pool's buffers move.
_POOL_TABLES: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()


def _pool_cache(pool) -> dict | None:
    try:
        return _POOL_TABLES.setdefault(pool, {})
    except TypeError:  # not weak-referenceable: build the table per call
        return None


def pool_rows(pool, *, index=None, block_table=None, page_size=None, index_offset: int = 0,
              head_offset: int = 0, tokens=None, pointer_cache: dict | None = None) -> Rows:
    """Describe any ``MHATokenToKVPool``-like object for the HIP kernels.

    A pool with one buffer per layer is described through a device table of
    layer pointers. Without ``pointer_cache`` the table is kept per pool, so
    it is uploaded once, not per call; launches record it on their stream.
    """
    if isinstance(pool, PagedKVPool):
        return pool.rows(index=index, block_table=block_table, page_size=page_size,
                         index_offset=index_offset, head_offset=head_offset, tokens=tokens)
    if pointer_cache is None:
        pointer_cache = _pool_cache(pool)
    layers = range(pool.start_layer, pool.start_layer + pool.layer_num)
    ks = [pool._get_key_buffer(l) for l in layers]
    vs = [pool._get_value_buffer(l) for l in layers]
    return rows_from_layers(ks, vs, index=index, block_table=block_table, page_size=page_size,
                            index_offset=index_offset, head_offset=head_offset, tokens=tokens,
                            pointer_cache=pointer_cache)
