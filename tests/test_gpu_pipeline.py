"""GPU: the two-stream staged layer-chunk pipeline installs exactly what the fused launch does.

Both paths run the same map kernel arithmetic per (target layer, head, kind),
so the target pools must be bit-identical, including rows outside each
sliding window (left untouched by both) and rows outside the request.
"""

from __future__ import annotations

import pytest
import torch

from cachebridge_amd import synthetic
from cachebridge_amd.online.pipeline import StagedHandoff
from cachebridge_amd.pool import pool_rows

pytestmark = pytest.mark.gpu


def _shape(name, tokens, layers):
    sh = synthetic.shape(name, tokens=tokens)
    sh.target_layers = layers
    if sh.windows is not None:
        sh.windows = sh.windows[:layers]
        sh.target_theta = sh.target_theta[:layers]
    return sh


@pytest.mark.parametrize("name,tokens,layers,chunk,blocks", [
    ("tp4", 700, 10, 4, [(0, 700)]),
    ("tp4", 700, 10, 3, [(0, 512), (512, 700)]),
    ("gemma", 1200, 12, 3, [(0, 1200)]),
])
def test_staged_pipeline_equals_fused_install(name, tokens, layers, chunk, blocks):
    print(f"staged pipeline {name} tokens={tokens} layers={layers} chunk={chunk} blocks={blocks}",
          flush=True)
    sh = _shape(name, tokens, layers)
    pages = (tokens + 15) // 16 * 3
    fused = synthetic.make_handoff(sh, target_pages=pages, fill_target="zeros")
    fused.run()
    staged_h = synthetic.make_handoff(sh, target_pages=pages, fill_target="zeros")
    width = max(b - a for a, b in blocks)
    staged = StagedHandoff(staged_h.mapper, layer_chunk=chunk, max_tokens=width)
    assert staged.staging_bytes == 2 * 2 * chunk * width * sh.target_heads * sh.head_dim * 2
    for start, stop in blocks:
        n = stop - start
        src = pool_rows(staged_h.source_pool, index=staged_h.source_slots, index_offset=start,
                        tokens=n)
        staged.run(src, staged_h.target_pool, num_tokens=n, position_start=start,
                   block_table=staged_h.block_table, page_size=16, index_offset=start,
                   prefix_length=tokens)
    torch.cuda.synchronize()
    for plan in staged.plans:
        assert plan.read_errors() == 0
    assert fused.mapper.plan.read_errors() == 0
    assert torch.equal(staged_h.target_pool.k_data, fused.target_pool.k_data)
    assert torch.equal(staged_h.target_pool.v_data, fused.target_pool.v_data)


def test_staged_pipeline_rejects_oversized_block():
    sh = _shape("tp4", 64, 2)
    h = synthetic.make_handoff(sh, target_pages=16, fill_target="zeros")
    staged = StagedHandoff(h.mapper, layer_chunk=2, max_tokens=32)
    src = pool_rows(h.source_pool, index=h.source_slots, tokens=64)
    with pytest.raises(ValueError, match="staging"):
        staged.run(src, h.target_pool, num_tokens=64, position_start=0,
                   block_table=h.block_table, page_size=16)
