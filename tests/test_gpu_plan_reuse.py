"""GPU: one plan launched with alternating shapes writes what fresh plans write.

A plan keeps the cost-line split of its last launch shape (blocks and
sub-tiles of each window class) and reuses it for the next launch of the same
shape. Launches that alternate between shapes (lengths, workgroup caps, window
mixes) must each write exactly the rows a plan that has never launched writes.
"""

from __future__ import annotations

import pytest
import torch

from cachebridge_amd import synthetic
from cachebridge_amd.online.blocks import map_install_block
from cachebridge_amd.pool import PagedKVPool

pytestmark = pytest.mark.gpu


def _empty_like(pool):
    return PagedKVPool(layer_num=pool.layer_num, pages=pool.pages, head_num=pool.head_num,
                       head_dim=pool.head_dim, page_size=pool.page_size, dtype=pool.dtype,
                       device=pool.device, fill="zeros")


@pytest.mark.parametrize("name,layers", [("tp4", 6), ("gemma", 12)])
def test_alternating_shapes_match_fresh_plans(name, layers):
    print(f"plan reuse {name} layers={layers}", flush=True)
    sh = synthetic.shape(name, tokens=3000)
    sh.target_layers = layers
    if sh.windows is not None:
        sh.windows = [None if w is None else 1024 for w in sh.windows[:layers]]
        sh.target_theta = sh.target_theta[:layers]
    h = synthetic.make_handoff(sh, fill_target="zeros")
    shapes = [(0, 3000, 0), (0, 700, 0), (0, 3000, 0), (0, 3000, 256), (500, 2100, 0), (0, 700, 0)]
    for start, stop, tpw in shapes:
        reused = _empty_like(h.target_pool)
        map_install_block(h.mapper, h.source_pool, h.source_slots, reused, start=start, stop=stop,
                          block_table=h.block_table, page_size=sh.page_size, prefix_length=3000,
                          tokens_per_workgroup=tpw)
        fresh_mapper = synthetic.make_mapper(sh, h.spec)
        fresh = _empty_like(h.target_pool)
        map_install_block(fresh_mapper, h.source_pool, h.source_slots, fresh, start=start, stop=stop,
                          block_table=h.block_table, page_size=sh.page_size, prefix_length=3000,
                          tokens_per_workgroup=tpw)
        torch.cuda.synchronize()
        assert h.mapper.plan.read_errors() == 0 and fresh_mapper.plan.read_errors() == 0
        assert torch.equal(reused.k_data, fresh.k_data), (start, stop, tpw)
        assert torch.equal(reused.v_data, fresh.v_data), (start, stop, tpw)
        del fresh_mapper
