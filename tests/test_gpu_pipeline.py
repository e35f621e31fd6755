"""GPU: the two-stream staged layer-chunk pipeline installs exactly what the fused launch does.

Both paths run the same map kernel arithmetic per (target layer, head, kind),
so the target pools must be bit-identical, including rows outside each
sliding window (left untouched by both) and rows outside the request. The
staged pipeline's own rows are also compared with the oracle on sampled token
windows (first, middle and last 64 tokens and both sides of each window
edge), every target layer, all heads, K and V, to the parity bar of
``oracle.tolerance.check_mapped``.
"""

from __future__ import annotations

import pytest
import torch

from cachebridge_amd import synthetic
from cachebridge_amd.online.pipeline import StagedHandoff
from cachebridge_amd.pool import pool_rows
from tests import fullsize as fs

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
    fs.fill_sentinel(fused.target_pool)
    fused.run()
    staged_h = synthetic.make_handoff(sh, target_pages=pages, fill_target="zeros")
    fs.fill_sentinel(staged_h.target_pool)
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
    assert torch.equal(staged_h.target_pool.k_data.view(torch.int16), fused.target_pool.k_data.view(torch.int16))
    assert torch.equal(staged_h.target_pool.v_data.view(torch.int16), fused.target_pool.v_data.view(torch.int16))

    dev = staged_h.target_pool.k_data.device
    tgt_slots = synthetic.slots_from_pages(staged_h.block_table.cpu(), tokens, 16).to(dev)
    first = fs.first_kept(sh.windows, sh.target_layers, prefix=tokens)
    stats = []
    for lo, hi in fs.token_windows(tokens, edges=sorted({f for f in first if f})):
        stats += fs.oracle_window(staged_h.source_pool, staged_h.source_slots, staged_h.target_pool,
                                  tgt_slots, staged_h.spec, lo=lo, hi=hi, position_start=0,
                                  layers=list(range(sh.target_layers)), source_theta=sh.source_theta,
                                  target_thetas=sh.target_theta, first=first)
    print("staged oracle", fs.summarize(stats), flush=True)


def test_staged_pipeline_rejects_oversized_block():
    sh = _shape("tp4", 64, 2)
    h = synthetic.make_handoff(sh, target_pages=16, fill_target="zeros")
    staged = StagedHandoff(h.mapper, layer_chunk=2, max_tokens=32)
    src = pool_rows(h.source_pool, index=h.source_slots, tokens=64)
    with pytest.raises(ValueError, match="staging"):
        staged.run(src, h.target_pool, num_tokens=64, position_start=0,
                   block_table=h.block_table, page_size=16)
