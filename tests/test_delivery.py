"""Receiver-side delivery geometry (CPU): run coalescing, spans and validation.

Follows ``rt/native_plan.py:1-95`` of the reference (``rt/`` =
``src/cachebridge/backends/sglang/runtime/``); the packed block the spans
describe is checked against the oracle's ``pack_source_block``
(``cb/online/blocks.py:47-82``), whose gather the reference tests pin.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cachebridge_amd.online.native_plan import Run, build_plan
from oracle import install as oi


def test_runs_coalesce_consecutive_rows_in_token_order():
    plan = build_plan([5, 6, 7, 20, 21, 3, 9, 10], start=1, stop=7, pool_rows=32, layers=3, heads=2,
                      dimension=4)
    assert plan.runs == (Run(6, 0, 2), Run(20, 2, 2), Run(3, 4, 1), Run(9, 5, 1))
    assert plan.useful_bytes == 2 * 3 * 6 * 2 * 4 * 2
    assert plan.copy_calls == 2 * 3 * 4
    single = build_plan(list(range(100, 164)), start=0, stop=64, pool_rows=200, layers=40)
    assert single.runs == (Run(100, 0, 64),) and single.copy_calls == 80


def test_spans_tile_the_packed_block_exactly():
    rng = np.random.default_rng(4)
    idx = [int(x) for x in rng.permutation(64)[:20]]
    idx[5:9] = [40, 41, 42, 43]
    plan = build_plan(idx, start=2, stop=18, pool_rows=64, layers=3, heads=2, dimension=8)
    row = 2 * 8 * 2
    covered = np.zeros(2 * 3 * 16 * row, dtype=np.int32)
    for s in plan.spans():
        covered[s["destination_byte_offset"]: s["destination_byte_offset"] + s["bytes"]] += 1
        assert s["source_byte_offset"] % row == 0 and s["bytes"] % row == 0
    assert covered.min() == 1 and covered.max() == 1


def test_span_copies_reproduce_the_oracle_pack():
    torch.manual_seed(0)
    layers, rows, heads, dim = 3, 48, 2, 8
    fill = torch.randn(2, layers, rows, heads, dim).to(torch.bfloat16)
    pool = oi.RowStorePool(layers, rows, heads, dim, fill=fill)
    idx = torch.tensor([7, 8, 9, 30, 2, 3, 4, 5, 40, 11], dtype=torch.int64)
    start, stop = 1, 9
    plan = build_plan(idx.tolist(), start=start, stop=stop, pool_rows=rows, layers=layers, heads=heads,
                      dimension=dim)
    packed = torch.zeros(2 * layers * (stop - start) * heads * dim, dtype=torch.bfloat16)
    dst = packed.view(torch.uint8)
    for s in plan.spans():
        buf = (pool._get_key_buffer if s["kind"] == 0 else pool._get_value_buffer)(s["layer"])
        src = buf.reshape(-1).view(torch.uint8)
        dst[s["destination_byte_offset"]: s["destination_byte_offset"] + s["bytes"]] = \
            src[s["source_byte_offset"]: s["source_byte_offset"] + s["bytes"]]
    workspace = torch.zeros(2 * layers * 16 * heads * dim, dtype=torch.bfloat16)
    ref = oi.pack_source_block(pool, idx, start=start, stop=stop, workspace=workspace, block_tokens=16)
    assert torch.equal(packed.view(2, layers, stop - start, heads, dim), ref)


def test_invalid_geometry_is_rejected():
    with pytest.raises(ValueError, match="integer geometry"):
        build_plan([1, 2], start=0, stop=2.0, pool_rows=4)
    with pytest.raises(ValueError, match="invalid geometry"):
        build_plan([1, 2], start=1, stop=1, pool_rows=4)
    with pytest.raises(ValueError, match="invalid geometry"):
        build_plan([1, 2], start=0, stop=2, pool_rows=4, element_bytes=4)
    with pytest.raises(ValueError, match="outside certified"):
        build_plan([1, 4], start=0, stop=2, pool_rows=4)
