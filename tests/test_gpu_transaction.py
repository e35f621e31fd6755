"""GPU: the unpublished install transaction over the fused map + install.

``install_unpublished`` (``cb/online/blocks.py:114-171``) is driven as the
reference's backend drives it: ``write`` enqueues one block's fused map +
install (``map_install_block``) on a side stream into pages the transaction
allocated, and ``synchronize`` is that stream's fence. Checked on the GPU:

- the request is published once, after the last block's write and fence and
  after the vote, with the stream idle at that moment;
- the published rows match the oracle and every other pool row is unchanged;
- a cancellation or a failed vote frees the allocated pages exactly once and
  publishes nothing; a vote that raises keeps them owned.
"""

from __future__ import annotations

import math
import time

import pytest
import torch

from cachebridge_amd import synthetic
from cachebridge_amd.online.blocks import install_unpublished, map_install_block
from tests import fullsize as fs

pytestmark = pytest.mark.gpu

TOKENS = 1024
BLOCK = 256
LAYERS = 8
PAGES = 256


class Transaction:
    """Callbacks of one target transaction over a shuffled free page list."""

    def __init__(self, h, stream, *, foreign_failure=False, vote_raises=False):
        self.h = h
        self.stream = stream
        self.events = []
        g = torch.Generator().manual_seed(9)
        self.free_pages = torch.randperm(PAGES, generator=g).tolist()
        self.foreign_failure = foreign_failure
        self.vote_raises = vote_raises
        self.table = None
        self.t_first_write = None
        self.t_publish = None

    def allocate(self, n):
        k = math.ceil(n / 16)
        pages, self.free_pages = self.free_pages[:k], self.free_pages[k:]
        self.table = torch.tensor(pages, dtype=torch.int32, device=self.h.target_pool.k_data.device)
        self.events.append(("allocate", k))
        return self.table

    def free(self, table):
        self.events.append(("free", table.data_ptr()))
        self.free_pages += table.tolist()

    def blocks(self):
        for start in range(0, TOKENS, BLOCK):
            stop = min(TOKENS, start + BLOCK)
            yield start, stop, self.h.source_slots[start:stop]

    def write(self, value, table, start):
        if self.t_first_write is None:
            self.t_first_write = time.perf_counter()
        stop = start + value.shape[0]
        map_install_block(self.h.mapper, self.h.source_pool, self.h.source_slots, self.h.target_pool,
                          start=start, stop=stop, block_table=table, page_size=16,
                          prefix_length=TOKENS, stream=self.stream)
        self.events.append(("write", start, stop))

    def synchronize(self):
        self.stream.synchronize()
        self.events.append(("sync",))

    def ready_vote(self, ok):
        self.events.append(("vote", ok))
        if self.vote_raises:
            raise RuntimeError("distributed group unavailable")
        return ok and not self.foreign_failure

    def publish(self, table):
        self.t_publish = time.perf_counter()
        self.events.append(("publish", table.data_ptr(), self.stream.query()))

    def run(self, **kw):
        return install_unpublished(token_count=TOKENS, allocate=self.allocate, free=self.free,
                                   blocks=self.blocks(), write=self.write,
                                   synchronize=self.synchronize, ready_vote=self.ready_vote,
                                   publish=self.publish, **kw)


def _handoff():
    sh = synthetic.shape("tp4", tokens=TOKENS)
    sh.target_layers = LAYERS
    h = synthetic.make_handoff(sh, target_pages=PAGES)
    fs.fill_sentinel(h.target_pool)
    return sh, h


def test_publish_after_every_block_is_installed():
    sh, h = _handoff()
    tx = Transaction(h, torch.cuda.Stream())
    result = tx.run()
    assert result == dict(tokens=TOKENS, blocks=TOKENS // BLOCK, published=True)
    kinds = [e[0] for e in tx.events]
    assert kinds == ["allocate"] + ["write", "sync"] * (TOKENS // BLOCK) + ["sync", "vote", "publish"]
    assert tx.events[-1][1] == tx.table.data_ptr() and tx.events[-1][2]  # stream idle at publish
    assert h.mapper.plan.read_errors() == 0
    print(f"first enqueue -> publish-ready: {1e3 * (tx.t_publish - tx.t_first_write):.3f} ms "
          f"({TOKENS} tokens, {TOKENS // BLOCK} blocks, {LAYERS} target layers)", flush=True)

    slots = synthetic.slots_from_pages(tx.table.cpu(), TOKENS, 16).to(tx.table.device)
    fs.check_untouched(h.target_pool, [slots] * LAYERS)
    stats = fs.oracle_window(h.source_pool, h.source_slots, h.target_pool, slots, h.spec, lo=0,
                             hi=TOKENS, position_start=0, layers=list(range(LAYERS)),
                             source_theta=sh.source_theta, target_thetas=sh.target_theta,
                             first=[0] * LAYERS)
    print("transaction oracle", fs.summarize(stats), flush=True)


@pytest.mark.parametrize("options", [dict(cancel_after_blocks=2), dict(foreign_failure=True)])
def test_cancel_or_failed_vote_frees_once_and_publishes_nothing(options):
    _, h = _handoff()
    cancel = options.pop("cancel_after_blocks", None)
    tx = Transaction(h, torch.cuda.Stream(), **options)
    with pytest.raises(RuntimeError, match="rolled back"):
        tx.run(cancel_after_blocks=cancel)
    kinds = [e[0] for e in tx.events]
    assert kinds.count("free") == 1 and "publish" not in kinds
    assert ("free", tx.table.data_ptr()) in tx.events
    assert kinds[-3:] == ["sync", "vote", "free"]
    assert len(tx.free_pages) == PAGES  # every page back on the free list
    assert h.mapper.plan.read_errors() == 0


def test_raising_vote_keeps_pages_owned():
    _, h = _handoff()
    tx = Transaction(h, torch.cuda.Stream(), vote_raises=True)
    with pytest.raises(RuntimeError, match="distributed group"):
        tx.run()
    kinds = [e[0] for e in tx.events]
    assert "free" not in kinds and "publish" not in kinds
    assert len(tx.free_pages) == PAGES - math.ceil(TOKENS / 16)
