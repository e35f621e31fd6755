"""GPU: block delivery of the selected source layers into two receiver slots.

Each block's slot equals the selected layers' source rows (bit for bit), and
mapping every delivered block (delivery and map on two streams, slots reused
after their map) installs exactly what the fused map from the source pool
installs.
"""

from __future__ import annotations

import pytest
import torch

from cachebridge_amd import synthetic
from cachebridge_amd.online.blocks import map_install_block
from cachebridge_amd.online.delivery import SelectedBlockDelivery, map_install_delivered

pytestmark = pytest.mark.gpu


def _shape(name, tokens, layers):
    sh = synthetic.shape(name, tokens=tokens)
    sh.target_layers = layers
    if sh.windows is not None:
        sh.windows = sh.windows[:layers]
        sh.target_theta = sh.target_theta[:layers]
    return sh


@pytest.mark.parametrize("name,tokens,layers,block,two_streams", [
    ("tp4", 1000, 8, 256, True),    # partial last block; slots reused across streams
    ("tp4", 1000, 8, 256, False),   # delivery and map on one stream
    ("tp4", 512, 4, 512, False),    # one block
    ("gemma", 1100, 12, 512, True),
])
def test_delivered_blocks_map_like_the_fused_install(name, tokens, layers, block, two_streams):
    print(f"delivery {name} tokens={tokens} layers={layers} block={block} two_streams={two_streams}",
          flush=True)
    sh = _shape(name, tokens, layers)
    pages = (tokens + 15) // 16 * 3
    fused = synthetic.make_handoff(sh, target_pages=pages, fill_target="zeros")
    map_install_block(fused.mapper, fused.source_pool, fused.source_slots, fused.target_pool, start=0,
                      stop=tokens, block_table=fused.block_table, page_size=16, prefix_length=tokens)
    h = synthetic.make_handoff(sh, target_pages=pages, fill_target="zeros")
    layers_sel = h.mapper.source_layers
    assert len(layers_sel) < sh.source_layers
    delivery = SelectedBlockDelivery(h.source_pool, h.source_slots, layers=layers_sel, block_tokens=block)
    compute = torch.cuda.Stream() if two_streams else torch.cuda.current_stream()
    for i, start in enumerate(range(0, tokens, block)):
        stop = min(start + block, tokens)
        view = delivery.deliver(i % 2, start, stop)
        with torch.cuda.stream(compute):
            map_install_delivered(h.mapper, delivery, i % 2, h.target_pool, block_table=h.block_table,
                                  page_size=16, prefix_length=tokens, stream=compute)
        if i == 0:
            delivery.stream.synchronize()
            rows = h.source_slots[start:stop].long()
            for p, l in enumerate(layers_sel):
                assert torch.equal(view[0, p], h.source_pool.k_buffer[l][rows])
                assert torch.equal(view[1, p], h.source_pool.v_buffer[l][rows])
    torch.cuda.synchronize()
    assert h.mapper.plan.read_errors() == 0 and fused.mapper.plan.read_errors() == 0
    assert torch.equal(h.target_pool.k_data, fused.target_pool.k_data)
    assert torch.equal(h.target_pool.v_data, fused.target_pool.v_data)
    r = delivery.receipt()
    assert r["launches"] == (tokens + block - 1) // block
    assert r["logical_input_bytes"] == 2 * len(layers_sel) * tokens * sh.source_heads * sh.head_dim * 2


def test_delivery_refuses_a_slot_still_in_use_and_bad_spans():
    sh = _shape("tp4", 300, 2)
    h = synthetic.make_handoff(sh, target_pages=64, fill_target="zeros")
    d = SelectedBlockDelivery(h.source_pool, h.source_slots, layers=h.mapper.source_layers, block_tokens=128)
    d.deliver(0, 0, 128)
    with pytest.raises(RuntimeError, match="unconsumed"):
        d.deliver(0, 128, 256)
    with pytest.raises(ValueError, match="invalid block span"):
        d.deliver(1, 0, 129)
    with pytest.raises(ValueError, match="source pool layers"):
        SelectedBlockDelivery(h.source_pool, h.source_slots, layers=[sh.source_layers], block_tokens=8)
    torch.cuda.synchronize()
