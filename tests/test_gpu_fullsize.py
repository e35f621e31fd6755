"""GPU: every configured workload at its full size, checked without a full-size oracle run.

Workloads (``cachebridge_amd.synthetic``):

- TP4 share: 40x2 -> 64x2, D 128, 4096 tokens into the 65,536-page pool;
- whole model, long history: 40x8 -> 64x8, 32,768 tokens;
- Gemma-style target: 62x16 with 52 sliding-window layers (window 1024) and
  10 global layers, 8192 tokens;
- 64 ragged requests (137,440 tokens) at the TP4 share into one pool at 85%
  occupancy;
- the shipped support-8 recipe's structure (every target layer reads 8 source
  layers, maps [1024, 128]) at the TP4 share and the whole model, 4096 tokens.

Each launch is checked for: error word 0; every pool row outside the
request's slots (and, per windowed layer, outside its window) bit-unchanged;
the rows equal, bit for bit, what the same work split into 2048-token blocks
(or, for the batch, one launch per request) writes; and the oracle at sampled
token windows (first, middle, last 64 tokens and both sides of each window
edge) for sampled target layers, all heads, K and V, to the parity bar of
``oracle.tolerance.check_mapped`` (1 bf16 ulp, or 2^-14 of the summand
magnitude for near-cancelling elements; >= 99.9% within 1 ulp; normwise
relative error <= 1e-2).
"""

from __future__ import annotations

import gc
import math

import pytest
import torch

from cachebridge_amd import synthetic
from cachebridge_amd.pool import pool_rows
from tests import fullsize as fs

pytestmark = pytest.mark.gpu

# Target layers sampled for the oracle: both ends, both sides of the middle,
# and a few in between; Gemma adds its first, middle and last global layers.
SAMPLE_64 = [0, 1, 17, 31, 32, 47, 62, 63]
SAMPLE_GEMMA = [0, 4, 5, 11, 30, 35, 59, 61]


@pytest.fixture(autouse=True)
def _release_memory():
    yield
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name,layers", [("tp4", SAMPLE_64), ("full32k", SAMPLE_64),
                                         ("gemma", SAMPLE_GEMMA), ("tp4_s8", SAMPLE_64),
                                         ("full_s8", SAMPLE_64)])
def test_full_size_handoff(name, layers):
    sh = synthetic.shape(name)
    t_count = sh.tokens
    print(f"full-size {name}: {sh.source_layers}x{sh.source_heads} -> "
          f"{sh.target_layers}x{sh.target_heads}, {t_count} tokens, {sh.target_pages} pages", flush=True)
    h = synthetic.make_handoff(sh, device_source=True)
    pool = h.target_pool
    dev = pool.k_data.device
    tgt_slots = synthetic.slots_from_pages(h.block_table.cpu(), t_count, sh.page_size).to(dev)
    first = fs.first_kept(sh.windows, sh.target_layers, prefix=t_count)
    written = [tgt_slots[f:] for f in first]

    fs.fill_sentinel(pool)
    h.run()
    assert h.mapper.plan.read_errors() == 0
    fs.check_untouched(pool, written)

    stats = []
    for lo, hi in fs.token_windows(t_count, edges=sorted({f for f in first if f})):
        stats += fs.oracle_window(h.source_pool, h.source_slots, pool, tgt_slots, h.spec, lo=lo,
                                  hi=hi, position_start=0, layers=layers,
                                  source_theta=sh.source_theta, target_thetas=sh.target_theta,
                                  first=first)
    print(name, "oracle", fs.summarize(stats), flush=True)

    single = fs.snapshot(pool, tgt_slots)
    fs.fill_sentinel(pool)
    for start in range(0, t_count, 2048):
        h.run(start=start, stop=min(t_count, start + 2048))
    assert h.mapper.plan.read_errors() == 0
    assert torch.equal(fs.snapshot(pool, tgt_slots), single)
    fs.check_untouched(pool, written)


@pytest.mark.parametrize("name", ["batch", "batch_full"])
def test_full_size_ragged_batch(name):
    """64 ragged requests in one launch: at the TP4 share into one pool at 85%
    occupancy, and at the whole-model 40x8 -> 64x8 geometry into a pool at
    50% occupancy (85% would need 260 GB next to the source pool)."""
    sh = synthetic.shape(name)
    b = synthetic.make_batch_handoff(sh)
    pool = b.target_pool
    dev = pool.k_data.device
    ps = sh.page_size
    print(f"full-size {name}: {len(b.lengths)} requests, {b.tokens} tokens, {sh.target_layers}x"
          f"{sh.target_heads}, {pool.pages} pages", flush=True)
    assert len(b.lengths) == 64
    src_of, tgt_of = [], []
    for sp in b.spans:
        e = sp.target_offset // ps
        pages = b.block_table[e:e + math.ceil(sp.num_tokens / ps)].cpu()
        tgt_of.append(synthetic.slots_from_pages(pages, sp.num_tokens, ps).to(dev))
        src_of.append(b.source_slots[sp.source_offset:sp.source_offset + sp.num_tokens])
    all_tgt = torch.cat(tgt_of)
    written = [all_tgt] * sh.target_layers

    fs.fill_sentinel(pool)
    b.run()
    assert b.mapper.plan.read_errors() == 0
    fs.check_untouched(pool, written)

    lengths = b.lengths
    order = sorted(range(len(lengths)), key=lambda i: lengths[i])
    g = torch.Generator().manual_seed(2024)
    picks = {order[0], order[-1], order[len(order) // 2]}
    picks.update(torch.randperm(len(lengths), generator=g)[:3].tolist())
    stats = []
    no_window = [0] * sh.target_layers
    for i in sorted(picks):
        sp = b.spans[i]
        for lo, hi in fs.token_windows(sp.num_tokens):
            stats += fs.oracle_window(b.source_pool, src_of[i], pool, tgt_of[i], b.spec, lo=lo,
                                      hi=hi, position_start=sp.position_start, layers=SAMPLE_64,
                                      source_theta=sh.source_theta, target_thetas=sh.target_theta,
                                      first=no_window)
    print(name, "oracle", sorted(picks), fs.summarize(stats), flush=True)

    batched = fs.snapshot(pool, all_tgt)
    fs.fill_sentinel(pool)
    for sp in b.spans:
        e = sp.target_offset // ps
        src = pool_rows(b.source_pool, index=b.source_slots, index_offset=sp.source_offset,
                        tokens=sp.num_tokens)
        tgt = pool_rows(pool, block_table=b.block_table[e:e + math.ceil(sp.num_tokens / ps)],
                        page_size=ps, tokens=sp.num_tokens)
        b.mapper.map_install(src, tgt, num_tokens=sp.num_tokens, position_start=sp.position_start,
                             prefix_length=sp.prefix_length)
    assert b.mapper.plan.read_errors() == 0
    assert torch.equal(fs.snapshot(pool, all_tgt), batched)
    fs.check_untouched(pool, written)
