"""GPU: the streaming kernel's work pool.

When a workgroup's share of a launch is long, the streaming kernel leaves the
tail of its work line to a pool of chunks that free workgroups claim from a
counter pair in plan-owned device memory; the launch's last workgroup clears
the pair, and a plan's direct launches rotate over 64 pairs (a launch whose
pair's previous launch still runs on another stream waits for it; bit 3 of
the error word would report a pair shared anyway). The whole 40x8 -> 64x8 model at
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
from cachebridge_amd.online.blocks import map_install_block
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
    if one stream ran 64 launches ahead. The library makes a launch wait for
    its pair's previous launch on another stream while that one runs, so every
    launch has its pair to itself: no error bit, every row installed."""
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
    assert h.mapper.plan.read_errors() == 0
    assert torch.equal(fs.snapshot(pool, slots), ref)


def test_pool_launches_64_apart_on_two_streams_install_both_requests():
    """Two requests of one plan, each a pooled launch capped to 32 workgroups
    (the TP4 share at 16,384 unit-tokens per workgroup), 64 apart in the
    plan's rotation and so on one counter pair, queued on two streams behind
    equal spin kernels so that both would start together; the 63 launches
    between them are unpooled ones of a third request on a third stream.
    Sharing the pair, the two launches would take chunk indices from one
    counter and each write some of the other's chunks with its own rows. The
    second launch must wait for the first instead: both requests' rows equal
    those of launches run one at a time, and no error bit is set."""
    sh = synthetic.shape("tp4")
    n = sh.tokens
    npages = (n + sh.page_size - 1) // sh.page_size
    print(f"two requests on one counter pair: {sh.target_layers}x{sh.target_heads}, {n} tokens each, "
          f"32 workgroups", flush=True)
    h = synthetic.make_handoff(sh, target_pages=4 * npages, device_source=True)
    pool = h.target_pool
    dev = pool.k_data.device
    g = torch.Generator().manual_seed(11)
    pages = torch.randperm(pool.pages, generator=g)[: 3 * npages].to(torch.int32)
    tables = [pages[i * npages:(i + 1) * npages].to(dev) for i in range(3)]
    slots = [synthetic.slots_from_pages(t.cpu(), n, sh.page_size).to(dev) for t in tables]

    def run(i, stream=None, cap=16384):
        map_install_block(h.mapper, h.source_pool, h.source_slots, pool, start=0, stop=n,
                          block_table=tables[i], page_size=sh.page_size, prefix_length=n,
                          stream=stream, tokens_per_workgroup=cap)

    fs.fill_sentinel(pool)
    run(0)
    assert h.mapper.plan.last_split() == (h.mapper.plan.last_split()[0], 32) and h.mapper.plan.last_split()[0] > 0
    run(1)
    assert h.mapper.plan.read_errors() == 0
    ref = [fs.snapshot(pool, slots[0]), fs.snapshot(pool, slots[1])]
    s1, s2, s3 = torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()
    # Several trials: whether two streams' launches run side by side depends
    # on how the runtime maps streams onto hardware queues and on first-use
    # costs (without the wait, a fresh process lost rows of both requests in
    # four of five trials).
    for trial in range(3):
        fs.fill_sentinel(pool)
        torch.cuda.synchronize()
        for s in (s1, s2):
            with torch.cuda.stream(s):
                torch.cuda._sleep(20_000_000)
        run(0, s1)
        for _ in range(63):
            run(2, s3, cap=0)
            assert h.mapper.plan.last_split()[0] == 0
        run(1, s2)
        torch.cuda.synchronize()
        assert h.mapper.plan.read_errors() == 0, f"trial {trial}"
        assert torch.equal(fs.snapshot(pool, slots[0]), ref[0]), f"trial {trial}: request A"
        assert torch.equal(fs.snapshot(pool, slots[1]), ref[1]), f"trial {trial}: request B"


def test_pool_launches_from_two_host_threads_install_both_requests():
    """Two host threads launch one plan concurrently, each 40 pooled launches
    (the TP4 share capped to 32 workgroups) of its own request on its own
    stream, so that launches 64 apart in the plan's rotation come from
    different threads and streams. Every launch must have its counter pair to
    itself: both requests' rows equal those of launches run one at a time, and
    no error bit is set."""
    import threading

    sh = synthetic.shape("tp4")
    n = sh.tokens
    npages = (n + sh.page_size - 1) // sh.page_size
    print(f"two host threads, one plan: {sh.target_layers}x{sh.target_heads}, {n} tokens each, "
          f"32 workgroups, 40 launches per thread", flush=True)
    h = synthetic.make_handoff(sh, target_pages=3 * npages, device_source=True)
    pool = h.target_pool
    dev = pool.k_data.device
    g = torch.Generator().manual_seed(13)
    pages = torch.randperm(pool.pages, generator=g)[: 2 * npages].to(torch.int32)
    tables = [pages[i * npages:(i + 1) * npages].to(dev) for i in range(2)]
    slots = [synthetic.slots_from_pages(t.cpu(), n, sh.page_size).to(dev) for t in tables]

    def run(i, stream=None):
        map_install_block(h.mapper, h.source_pool, h.source_slots, pool, start=0, stop=n,
                          block_table=tables[i], page_size=sh.page_size, prefix_length=n,
                          stream=stream, tokens_per_workgroup=16384)

    fs.fill_sentinel(pool)
    run(0)
    run(1)
    assert h.mapper.plan.last_split()[0] > 0
    assert h.mapper.plan.read_errors() == 0
    ref = [fs.snapshot(pool, slots[0]), fs.snapshot(pool, slots[1])]
    fs.fill_sentinel(pool)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    errors = []

    def worker(i):
        try:
            with torch.cuda.device(dev):
                for _ in range(40):
                    run(i, streams[i])
        except Exception as exc:  # noqa: BLE001 -- reported by the main thread
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    assert h.mapper.plan.read_errors() == 0
    assert torch.equal(fs.snapshot(pool, slots[0]), ref[0])
    assert torch.equal(fs.snapshot(pool, slots[1]), ref[1])
