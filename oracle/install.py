"""Oracle restatement of the gather / map / paged-install path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

- ``RowStorePool``: SGLang ``MHATokenToKVPool`` duck type (``layer_num``,
  ``start_layer``, ``dtype``, ``_get_key_buffer``, ``_get_value_buffer``,
  ``set_kv_buffer``) as consumed at ``cb/online/blocks.py:57-59,79-81,106-111``
  and ``cb/backends/sglang/runtime/r010_core.py:37-43``. SGLang v0.4.10.post2
  (commit 8cd344586e09669432d35c678b7cc208c0a6f47e) is an un-vendored
  dependency; its ``set_kv_buffer`` is restated as a plain row store
  ``buffer[layer][loc] = k.to(dtype)``. SGLang's own code is not available
  here. The restatement is pinned by the check the reference runs after its
  installs through SGLang's pool (``rt/clean_adapter.py:638-652``: the rows at
  ``indices`` of every layer bit-equal the written values) and by the
  row-store invariant that every other row is unchanged
  (``tests/test_oracle.py``).
- ``pack_source_block`` / ``map_write_block``: ``cb/online/blocks.py:47-111``.
  Pinned by ``tests/test_blocks.py:33-65`` of the reference (restated as a test).
- ``virtual_source_page``: re-index a source pool into a page whose layer
  ``l*s+k`` holds, for every target head ``h``, the assigned source
  ``(layer, head)`` pair ``k`` of target ``(l, h)``. With ``selected[l] =
  [l*s+k for k]`` the reference mapper then computes exactly the map for an
  arbitrary per-(layer, head) source assignment (un-rotation is elementwise
  per position, so re-indexing before it is exact). Pinned by the identity
  ``virtual page == reference page`` for head-identity assignments.
- ``materialize_window``: ``cb/architectures/gemma3.py:39-58``. Pinned by the
  reference test ``tests/test_architectures.py:126-144`` (restated).
"""

from __future__ import annotations

from types import SimpleNamespace

import torch
from torch import Tensor

from .mapper import PageMapper


class RowStorePool:
    """Per-layer ``[rows, heads, head_dim]`` K and V buffers with row-store install."""

    def __init__(self, layers: int, rows: int, heads: int, head_dim: int,
                 dtype=torch.bfloat16, start_layer: int = 0, fill: Tensor | None = None):
        self.layer_num = layers
        self.start_layer = start_layer
        self.dtype = dtype
        self.k_buffer = [torch.zeros(rows, heads, head_dim, dtype=dtype) for _ in range(layers)]
        self.v_buffer = [torch.zeros(rows, heads, head_dim, dtype=dtype) for _ in range(layers)]
        if fill is not None:
            for i in range(layers):
                self.k_buffer[i].copy_(fill[0, i])
                self.v_buffer[i].copy_(fill[1, i])

    def _get_key_buffer(self, layer: int) -> Tensor:
        return self.k_buffer[layer - self.start_layer]

    def _get_value_buffer(self, layer: int) -> Tensor:
        return self.v_buffer[layer - self.start_layer]

    def set_kv_buffer(self, layer, loc, cache_k, cache_v, layer_id_override=None):
        index = layer_id_override if layer_id_override is not None else layer.layer_id
        if cache_k.dtype != self.dtype:
            cache_k = cache_k.to(self.dtype)
            cache_v = cache_v.to(self.dtype)
        self.k_buffer[index - self.start_layer][loc] = cache_k
        self.v_buffer[index - self.start_layer][loc] = cache_v


@torch.inference_mode()
def pack_source_block(pool, indices, *, start, stop, workspace, block_tokens):
    """``cb/online/blocks.py:47-82``: gather pool rows into one contiguous block."""
    n = stop - start
    if not 0 <= start < stop <= len(indices) or n > block_tokens:
        raise ValueError("invalid block span")
    layers = pool.layer_num
    first = pool._get_key_buffer(pool.start_layer)
    heads, dim = first.shape[1:]
    if (workspace.ndim != 1 or workspace.numel() != 2 * layers * block_tokens * heads * dim
            or not workspace.is_contiguous()):
        raise ValueError("workspace must be exactly one contiguous block")
    if (workspace.device != first.device or workspace.dtype != first.dtype
            or indices.device != first.device):
        raise ValueError("pool, indices and workspace must share device and dtype as applicable")
    if indices.ndim != 1 or indices.dtype not in (torch.int32, torch.int64):
        raise ValueError("one-dimensional integer pool indices required")
    block = workspace[: 2 * layers * n * heads * dim].view(2, layers, n, heads, dim)
    loc = indices[start:stop]
    for i in range(layers):
        layer = pool.start_layer + i
        torch.index_select(pool._get_key_buffer(layer), 0, loc, out=block[0, i])
        torch.index_select(pool._get_value_buffer(layer), 0, loc, out=block[1, i])
    return block


@torch.inference_mode()
def map_write_block(mapper, block, target_pool, target_indices, *, start, source_head_offset):
    """``cb/online/blocks.py:86-111``: map one block and row-store it per target layer."""
    n = block.shape[2]
    if start < 0 or start + n > len(target_indices) or mapper.method != "cachebridge":
        raise ValueError("invalid target range or non-CacheBridge method")
    device = target_pool._get_key_buffer(target_pool.start_layer).device
    mapped = mapper.map_page(block, position_start=start,
                             source_head_offset=source_head_offset, output_device=device)
    if mapped.shape[:3] != (2, target_pool.layer_num, n) or mapped.dtype != target_pool.dtype:
        raise ValueError("mapper output geometry/dtype mismatch")
    loc = target_indices[start: start + n]
    for i in range(target_pool.layer_num):
        layer = target_pool.start_layer + i
        target_pool.set_kv_buffer(None, loc, mapped[0, i], mapped[1, i], layer_id_override=layer)


def virtual_source_page(source_page: Tensor, assign_layer: Tensor, assign_head: Tensor,
                        source_head_offset: int = 0) -> Tensor:
    """Re-index ``[2, Ls, n, Hs, D]`` into ``[2, Lt*s, n, Ht, D]`` by assignment.

    ``assign_layer``/``assign_head`` are ``[Lt, Ht, s]`` integer tensors of global
    source indices; page head ``h - source_head_offset`` holds global head ``h``.
    """
    lt, ht, s = assign_layer.shape
    out = source_page.new_empty(2, lt * s, source_page.shape[2], ht, source_page.shape[4])
    for l in range(lt):
        for h in range(ht):
            for k in range(s):
                sl = int(assign_layer[l, h, k])
                sh = int(assign_head[l, h, k]) - source_head_offset
                if not 0 <= sh < source_page.shape[3] or not 0 <= sl < source_page.shape[1]:
                    raise ValueError("assigned source (layer, head) is not in the page")
                out[:, l * s + k, :, h] = source_page[:, sl, :, sh]
    return out


def assignment_mapper(spec: dict, layers: list[int] | None = None, *, source_rope_theta,
                      target_rope_theta, source_rope_scaling=None, target_rope_scaling=None,
                      device="cpu") -> PageMapper:
    """Reference mapper over the virtual page for target layers ``layers``.

    ``spec`` holds ``assign_layer``/``assign_head`` ``[Lt, Ht, s]`` and
    ``k_weight``/``v_weight`` ``[Lt, Ht, s*D, D]``, ``k_bias``/``v_bias``
    ``[Lt, Ht, D]`` (fp32). Layer ``i`` of the returned mapper is target layer
    ``layers[i]`` and selects virtual layers ``layers[i]*s + k``.
    """
    lt, _, s = spec["assign_layer"].shape
    layers = list(range(lt)) if layers is None else layers
    tensors = []
    for l in layers:
        tensors.append({
            "selected": torch.tensor([l * s + k for k in range(s)], dtype=torch.int64),
            "k_weight": spec["k_weight"][l], "k_bias": spec["k_bias"][l],
            "v_weight": spec["v_weight"][l], "v_bias": spec["v_bias"][l],
            "headwise": torch.tensor(1, dtype=torch.int8),
        })
    return PageMapper.from_tensors(
        tensors, method="cachebridge", source_rope_theta=source_rope_theta,
        target_rope_theta=target_rope_theta, source_rope_scaling=source_rope_scaling,
        target_rope_scaling=target_rope_scaling, device=device,
    )


def materialize_window(tokens: int, *, layer_type: str, sliding_window) -> int:
    """``cb/architectures/gemma3.py:39-58``: first retained token of a layer.

    Sliding layers keep the last ``min(tokens, sliding_window - 1)`` tokens;
    full-attention layers keep all of them.
    """
    if tokens < 1:
        raise ValueError("prefix length must equal the materialized token count")
    if layer_type == "sliding_attention":
        if int(sliding_window) < 2:
            raise ValueError("Sliding window must leave room for the next token")
        retained = min(tokens, int(sliding_window) - 1)
    elif layer_type == "full_attention":
        retained = tokens
    else:
        raise ValueError(f"Unsupported Gemma layer type: {layer_type}")
    return tokens - retained


@torch.inference_mode()
def map_install_oracle(source_pool, source_slots: Tensor, target_pool: RowStorePool,
                       target_slots: Tensor, spec: dict, *, position_start: int,
                       source_theta: float, target_thetas, windows=None,
                       prefix_length: int | None = None, source_scaling=None,
                       target_scaling=None, source_head_offset: int = 0) -> Tensor:
    """Whole-path oracle: gather, map (per target-theta/window group), row-store install.

    ``source_slots``/``target_slots`` give the pool row of each of the block's
    ``n`` tokens. ``target_thetas`` is a per-target-layer list; ``windows`` a
    per-target-layer list of ``None`` (full attention) or a sliding-window size,
    applied against ``prefix_length`` (default: ``position_start + n``). Returns
    the mapped ``[2, Lt, n, Ht, D]`` tensor (all tokens, before windowing).
    """
    n = int(source_slots.numel())
    lt = spec["assign_layer"].shape[0]
    pool_view = SimpleNamespace(
        layer_num=source_pool.layer_num, start_layer=source_pool.start_layer,
        _get_key_buffer=source_pool._get_key_buffer,
        _get_value_buffer=source_pool._get_value_buffer,
    )
    first = source_pool._get_key_buffer(source_pool.start_layer)
    workspace = torch.empty(2 * source_pool.layer_num * n * first.shape[1] * first.shape[2],
                            dtype=first.dtype)
    page = pack_source_block(pool_view, source_slots, start=0, stop=n,
                             workspace=workspace, block_tokens=n)
    virtual = virtual_source_page(page, spec["assign_layer"], spec["assign_head"],
                                  source_head_offset)
    thetas = list(target_thetas) if not isinstance(target_thetas, (int, float)) else [target_thetas] * lt
    ht, dim = spec["k_bias"].shape[1], spec["k_bias"].shape[2]
    mapped = torch.empty(2, lt, n, ht, dim, dtype=first.dtype)
    for theta in sorted(set(thetas)):
        group = [l for l in range(lt) if thetas[l] == theta]
        mapper = assignment_mapper(spec, group, source_rope_theta=source_theta,
                                   target_rope_theta=theta, source_rope_scaling=source_scaling,
                                   target_rope_scaling=target_scaling)
        out = mapper.map_page(virtual, position_start=position_start)
        for i, l in enumerate(group):
            mapped[:, l] = out[:, i]
    prefix = position_start + n if prefix_length is None else prefix_length
    for l in range(lt):
        first_pos = 0
        if windows is not None and windows[l] is not None:
            first_pos = materialize_window(prefix, layer_type="sliding_attention",
                                           sliding_window=windows[l])
        keep = max(0, first_pos - position_start)
        if keep >= n:
            continue
        target_pool.set_kv_buffer(None, target_slots[keep:], mapped[0, l, keep:],
                                  mapped[1, l, keep:], layer_id_override=target_pool.start_layer + l)
    return mapped
