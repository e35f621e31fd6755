"""Receiver-side delivery geometry (CPU): runs of consecutive source rows.

A block's slot indices split into maximal runs of consecutive physical rows
(the unit of the reference's span-by-span peer copies,
``rt/native_plan.py:58-95`` with ``rt/`` =
``src/cachebridge/backends/sglang/runtime/``). Checked here: the runs tile
the block in token order, and copying them run by run into a packed
``[2, layers, n, heads, dim]`` block reproduces the oracle's
``pack_source_block`` (``cb/online/blocks.py:47-82``), whose gather the
reference tests pin.
"""

from __future__ import annotations

import numpy as np
import torch

from cachebridge_amd.online.delivery import coalesced_runs
from oracle import install as oi


def brute_runs(rows):
    out = []
    for t, r in enumerate(rows):
        if out and r == rows[t - 1] + 1:
            out[-1][1] += 1
        else:
            out.append([t, 1])
    return out


def test_runs_match_a_brute_force_scan():
    rng = np.random.default_rng(4)
    cases = [[5, 6, 7, 20, 21, 3, 9, 10], list(range(100, 164)), [7], [3, 2, 1], [],
             [int(x) for x in rng.permutation(64)[:40]]]
    for rows in cases:
        first, length = coalesced_runs(torch.tensor(rows, dtype=torch.int32))
        assert [[int(a), int(b)] for a, b in zip(first, length)] == brute_runs(rows)
    first, length = coalesced_runs(torch.tensor([6, 7, 20, 21, 3, 9]))
    assert first.tolist() == [0, 2, 4, 5] and length.tolist() == [2, 2, 1, 1]


def test_run_copies_reproduce_the_oracle_pack():
    torch.manual_seed(0)
    layers, rows, heads, dim = 3, 48, 2, 8
    fill = torch.randn(2, layers, rows, heads, dim).to(torch.bfloat16)
    pool = oi.RowStorePool(layers, rows, heads, dim, fill=fill)
    idx = torch.tensor([7, 8, 9, 30, 2, 3, 4, 5, 40, 11], dtype=torch.int64)
    start, stop = 1, 9
    n = stop - start
    packed = torch.zeros(2, layers, n, heads, dim, dtype=torch.bfloat16)
    first, length = coalesced_runs(idx[start:stop])
    assert int(length.sum()) == n
    for kind, get in enumerate((pool._get_key_buffer, pool._get_value_buffer)):
        for layer in range(layers):
            for t, m in zip(first.tolist(), length.tolist()):
                row = int(idx[start + t])
                packed[kind, layer, t:t + m] = get(layer)[row:row + m]
    workspace = torch.zeros(2 * layers * 16 * heads * dim, dtype=torch.bfloat16)
    ref = oi.pack_source_block(pool, idx, start=start, stop=stop, workspace=workspace, block_tokens=16)
    assert torch.equal(packed, ref)
