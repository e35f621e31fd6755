"""GPU: a ragged batch of requests in one launch installs exactly what per-request launches do.

Each request of the batch has its own source slots, block-table pages,
positions and prefix (windows). The batch writes every row bit-identically
to one ``map_install`` per request (the per-request path is pinned against
the oracle by the fused-install parity tests), leaves every other row
untouched, and flags rows an index places outside a pool without writing
them.
"""

from __future__ import annotations

import pytest
import torch

from cachebridge_amd import synthetic
from cachebridge_amd.online.blocks import map_install_batch
from cachebridge_amd.plan import RequestSpan
from cachebridge_amd.pool import PagedKVPool, pool_rows

pytestmark = pytest.mark.gpu


def _shape(name, tokens, layers):
    sh = synthetic.shape(name, tokens=tokens)
    if layers is not None:
        sh.target_layers = layers
        if sh.windows is not None:
            sh.windows = [None if w is None else 1024 for w in sh.windows[:layers]]
            sh.target_theta = sh.target_theta[:layers]
    return sh


def _batch(lengths, positions, prefixes, pages_total, seed):
    """Spans over one concatenated source-slot vector and one concatenated block table."""
    g = torch.Generator().manual_seed(seed)
    order = torch.randperm(pages_total, generator=g).to(torch.int32)
    spans, src, entry = [], 0, 0
    for n, p, pre in zip(lengths, positions, prefixes):
        spans.append(RequestSpan(src, entry * 16, n, p, pre))
        src += n
        entry += (n + 15) // 16
    assert entry <= pages_total
    return spans, order[:max(entry, 1)].contiguous()


def _target_like(pool, fill="zeros"):
    return PagedKVPool(layer_num=pool.layer_num, pages=pool.pages, head_num=pool.head_num,
                       head_dim=pool.head_dim, page_size=pool.page_size, dtype=pool.dtype,
                       device=pool.device, fill=fill)


@pytest.mark.parametrize("name,layers,lengths,positions,prefixes", [
    ("tp4", 6, [1, 15, 0, 16, 17, 300, 1000, 2500], [0, 0, 0, 3, 40, 0, 77, 0], [0] * 8),
    ("toy", None, [5, 64, 200, 33], [0, 10, 0, 100], [0, 0, 0, 0]),
    ("gemma", 12, [200, 1500, 700, 2100], [0, 0, 500, 0], [0, 0, 2000, 0]),
])
def test_batch_equals_per_request_installs(name, layers, lengths, positions, prefixes):
    print(f"batch {name} layers={layers} lengths={lengths}", flush=True)
    sh = _shape(name, sum(lengths), layers)
    pages = sum((n + 15) // 16 for n in lengths) * 2
    h = synthetic.make_handoff(sh, target_pages=pages, fill_target="zeros")
    spans, bt = _batch(lengths, positions, prefixes, pages, seed=11)
    check_batch_equals_single(h, spans, bt.to(h.target_pool.device))


def check_batch_equals_single(h, spans, bt):
    """One batched launch over ``spans`` against one ``map_install`` per request."""
    map_install_batch(h.mapper, h.source_pool, h.source_slots, h.target_pool, spans,
                      block_table=bt, page_size=16)
    assert h.mapper.plan.read_errors() == 0
    single = _target_like(h.target_pool)
    for sp in spans:
        if sp.num_tokens == 0:
            continue
        e = sp.target_offset // 16
        src = pool_rows(h.source_pool, index=h.source_slots, index_offset=sp.source_offset,
                        tokens=sp.num_tokens)
        tgt = pool_rows(single, block_table=bt[e:e + (sp.num_tokens + 15) // 16], page_size=16,
                        tokens=sp.num_tokens)
        h.mapper.map_install(src, tgt, num_tokens=sp.num_tokens, position_start=sp.position_start,
                             prefix_length=sp.prefix_length)
    torch.cuda.synchronize()
    assert h.mapper.plan.read_errors() == 0
    assert torch.equal(h.target_pool.k_data, single.k_data)
    assert torch.equal(h.target_pool.v_data, single.v_data)
    # the batch wrote the last token of every request that some layer keeps
    # (so the comparison is not between two all-zero pools)
    for sp in spans:
        if sp.num_tokens and _some_layer_keeps_last_token(h.shape, sp):
            u = sp.target_offset + sp.num_tokens - 1
            row = int(bt[u // 16]) * 16 + u % 16
            assert h.target_pool.v_data[:, row].abs().sum() > 0


def _some_layer_keeps_last_token(sh, sp):
    """A layer without a window keeps every token; a window W keeps the last W - 1 of the prefix."""
    prefix = sp.prefix_length or sp.position_start + sp.num_tokens
    last = sp.position_start + sp.num_tokens - 1
    return any(w is None or last >= prefix - (w - 1) for w in (sh.windows or [None]))


def test_batch_flags_out_of_range_rows_and_skips_them():
    sh = _shape("tp4", 96, 2)
    h = synthetic.make_handoff(sh, target_pages=16, fill_target="zeros")
    spans, bt = _batch([40, 56], [0, 0], [0, 0], 16, seed=3)
    bt = bt.to(h.target_pool.device)
    bad = bt.clone()
    bad[1] = h.target_pool.pages + 5  # request 0's second page lies beyond the pool
    map_install_batch(h.mapper, h.source_pool, h.source_slots, h.target_pool, spans,
                      block_table=bad, page_size=16)
    assert h.mapper.plan.read_errors() & 2
    good = _target_like(h.target_pool)
    # request 0 without its tokens 16..31 (the bad page): those rows are not written
    ok = [spans[0]._replace(num_tokens=16),
          RequestSpan(spans[0].source_offset + 32, spans[0].target_offset + 32, 8, 32, 40),
          spans[1]]
    map_install_batch(h.mapper, h.source_pool, h.source_slots, good, ok, block_table=bt,
                      page_size=16)
    assert h.mapper.plan.read_errors() == 0
    assert torch.equal(h.target_pool.k_data, good.k_data)
    assert torch.equal(h.target_pool.v_data, good.v_data)


def test_batch_rejects_bad_requests_before_launch():
    sh = _shape("tp4", 64, 2)
    h = synthetic.make_handoff(sh, target_pages=16, fill_target="zeros")
    spans, bt = _batch([32, 32], [0, 0], [0, 0], 16, seed=5)
    bt = bt.to(h.target_pool.device)
    with pytest.raises(ValueError, match="positions"):
        map_install_batch(h.mapper, h.source_pool, h.source_slots, h.target_pool,
                          [spans[0]._replace(position_start=h.mapper.plan.max_positions - 8)],
                          block_table=bt, page_size=16)
    with pytest.raises(ValueError, match="source_indices"):
        map_install_batch(h.mapper, h.source_pool, h.source_slots, h.target_pool,
                          [spans[1]._replace(source_offset=40)], block_table=bt, page_size=16)
    with pytest.raises(ValueError, match="block table"):
        map_install_batch(h.mapper, h.source_pool, h.source_slots, h.target_pool,
                          [spans[1]._replace(target_offset=16 * 16)], block_table=bt, page_size=16)
    with pytest.raises(ValueError, match="prefix_length"):
        map_install_batch(h.mapper, h.source_pool, h.source_slots, h.target_pool,
                          [spans[0]._replace(prefix_length=10)], block_table=bt, page_size=16)
    torch.cuda.synchronize()
    assert int(h.target_pool.k_data.abs().sum()) == 0  # nothing was written
    map_install_batch(h.mapper, h.source_pool, h.source_slots, h.target_pool, [],
                      block_table=bt, page_size=16)  # an empty batch is a no-op
