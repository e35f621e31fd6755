"""GPU: the streaming kernel's work pool.

When a workgroup's share of a launch is long, the streaming kernel leaves the
tail of its work line to a pool of chunks that free workgroups claim from a
counter pair in plan-owned device memory; the launch's last workgroup clears
the pair, and a plan's direct launches rotate over 64 pairs (a launch that
finds its pair shared sets bit 3 of the error word). The whole 40x8 -> 64x8 model at
4096 tokens is such a launch (about 13K weight units of work per workgroup,
above the pool threshold of 8192); 512-token launches of the same work are
not (below 2K). These tests check that every launch of a pooled shape
installs every row, across more launches than the plan has counter pairs and
with launches overlapping on two streams.
"""

from __future__ import annotations

import gc

import pytest
import torch

from cachebridge_amd import synthetic
from tests import fullsize as fs

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _release_memory():
    yield
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def test_pool_installs_every_row_over_many_launches():
    sh = synthetic.shape("full")
    n = sh.tokens
    print(f"pooled handoff: {sh.source_layers}x{sh.source_heads} -> {sh.target_layers}x{sh.target_heads}, "
          f"{n} tokens, 512 target pages", flush=True)
    h = synthetic.make_handoff(sh, target_pages=512, device_source=True)
    pool = h.target_pool
    slots = synthetic.slots_from_pages(h.block_table.cpu(), n, sh.page_size).to(pool.k_data.device)
    written = [slots] * sh.target_layers

    fs.fill_sentinel(pool)
    h.run()
    assert h.mapper.plan.read_errors() == 0
    assert h.mapper.plan.last_split()[0] > 0, "the 4096-token whole-model launch must use the pool"
    fs.check_untouched(pool, written)
    ref = fs.snapshot(pool, slots)

    # Launches overlapping on two streams take different counter pairs.
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for _ in range(8):
        h.run(stream=s1)
        h.run(stream=s2)
    torch.cuda.synchronize()
    assert torch.equal(fs.snapshot(pool, slots), ref)

    # Every counter pair then serves two more launches; each must install
    # every row (a pair left non-zero would make its next launch skip chunks,
    # leaving sentinel rows).
    for i in range(2 * 64 + 3):
        fs.fill_sentinel(pool)
        h.run()
        assert torch.equal(fs.snapshot(pool, slots), ref), f"launch {i} after the overlapping ones"
    assert h.mapper.plan.read_errors() == 0

    # 512-token launches (no pool) write the same rows bit for bit.
    fs.fill_sentinel(pool)
    for start in range(0, n, 512):
        h.run(start=start, stop=min(n, start + 512))
        assert h.mapper.plan.last_split()[0] == 0
    assert h.mapper.plan.read_errors() == 0
    assert torch.equal(fs.snapshot(pool, slots), ref)
    fs.check_untouched(pool, written)


def test_pool_on_a_capped_grid_matches_the_full_grid():
    """A cap on tokens per workgroup shrinks the grid: the TP4 share at 4096
    tokens with 16,384 unit-tokens per workgroup runs on 32 workgroups, each
    with about 26K weight units of work (a pool), where the default grid of
    256 has about 3.2K (no pool). Both write the same rows bit for bit."""
    sh = synthetic.shape("tp4")
    n = sh.tokens
    print(f"capped grid: {sh.target_layers}x{sh.target_heads}, {n} tokens, 16384 unit-tokens per workgroup",
          flush=True)
    h = synthetic.make_handoff(sh, target_pages=1024, device_source=True)
    pool = h.target_pool
    slots = synthetic.slots_from_pages(h.block_table.cpu(), n, sh.page_size).to(pool.k_data.device)
    written = [slots] * sh.target_layers

    fs.fill_sentinel(pool)
    h.run()
    assert h.mapper.plan.read_errors() == 0
    assert h.mapper.plan.last_split()[0] == 0
    ref = fs.snapshot(pool, slots)
    for i in range(3):
        fs.fill_sentinel(pool)
        h.run(tokens_per_workgroup=16384)
        chunks, groups = h.mapper.plan.last_split()
        assert chunks > 0 and groups == 32, (chunks, groups)
        assert h.mapper.plan.read_errors() == 0
        assert torch.equal(fs.snapshot(pool, slots), ref), f"capped launch {i}"
    fs.check_untouched(pool, written)


def test_pool_launches_queued_on_three_streams():
    """150 pooled launches queued round-robin on three streams, without
    waiting: launch k uses counter pair k % 64 and lands on stream k % 3, so
    launches 64 apart sit on different streams and could run at the same time
    if one stream ran 64 launches ahead. Every launch must then either have
    had its pair to itself and written every row, or report the sharing in
    bit 3 of the error word: rows may never go missing silently."""
    sh = synthetic.shape("full")
    n = sh.tokens
    print(f"three-stream pooled launches: {sh.target_layers}x{sh.target_heads}, {n} tokens", flush=True)
    h = synthetic.make_handoff(sh, target_pages=512, device_source=True)
    pool = h.target_pool
    slots = synthetic.slots_from_pages(h.block_table.cpu(), n, sh.page_size).to(pool.k_data.device)
    fs.fill_sentinel(pool)
    h.run()
    assert h.mapper.plan.read_errors() == 0
    assert h.mapper.plan.last_split()[0] > 0
    ref = fs.snapshot(pool, slots)
    streams = [torch.cuda.Stream() for _ in range(3)]
    fs.fill_sentinel(pool)
    torch.cuda.synchronize()
    for k in range(150):
        h.run(stream=streams[k % 3])
    torch.cuda.synchronize()
    flags = h.mapper.plan.read_errors()
    assert flags & ~8 == 0, flags
    if not flags & 8:
        assert torch.equal(fs.snapshot(pool, slots), ref)
