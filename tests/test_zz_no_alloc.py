"""GPU: the no-allocation batched install writes exactly what the allocating one writes.

``cb_map_install_batch_noalloc`` is called through the C ABI on two ragged
batches in a row, the second smaller than the first (so stale workspace
contents from the first call would show), and each result is compared bit for
bit with ``cb_map_install_batch`` given a torch-allocated workspace (that path
is pinned against the oracle by the batch and full-size tests). A batch long
enough for the streaming kernel's work pool runs the same way, twice around a
short one. A batch beyond the fixed workspace is rejected before anything is
enqueued.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from cachebridge_amd import _lib, synthetic
from cachebridge_amd.plan import RequestSpan, _span_array
from cachebridge_amd.pool import PagedKVPool, pool_rows

pytestmark = pytest.mark.gpu


def _spans(lengths, positions, pages_total, seed):
    g = torch.Generator().manual_seed(seed)
    order = torch.randperm(pages_total, generator=g).to(torch.int32)
    spans, src, entry = [], 0, 0
    for n, p in zip(lengths, positions):
        spans.append(RequestSpan(src, entry * 16, n, p, 0))
        src += n
        entry += (n + 15) // 16
    assert entry <= pages_total
    return spans, order[:entry].contiguous()


def _zero_pool_like(pool):
    return PagedKVPool(layer_num=pool.layer_num, pages=pool.pages, head_num=pool.head_num,
                       head_dim=pool.head_dim, page_size=pool.page_size, dtype=pool.dtype,
                       device=pool.device, fill="zeros")


@pytest.mark.parametrize("workload", ["tp4", "tp4_s8"])
def test_noalloc_batch_equals_allocating_batch_on_two_calls(workload):
    """Both map kernels a batch can use: the streaming kernel (support 1) and
    the support kernel (support 8)."""
    lib = _lib.load()
    batches = [([700, 1, 300, 1500, 17, 900, 64], [0, 5, 0, 40, 0, 100, 7]),
               ([200, 33], [0, 3])]
    tokens = sum(batches[0][0])
    sh = synthetic.shape(workload, tokens=tokens)
    sh.target_layers = 6
    pages = sum((n + 15) // 16 for n in batches[0][0]) * 2
    h = synthetic.make_handoff(sh, target_pages=pages, fill_target="zeros")
    plan = h.mapper.plan
    stream = torch.cuda.current_stream()
    for call, (lengths, positions) in enumerate(batches):
        print(f"no-alloc {workload} call {call}: {len(lengths)} requests, {sum(lengths)} tokens", flush=True)
        spans, bt = _spans(lengths, positions, pages, seed=20 + call)
        bt = bt.to(h.target_pool.device)
        want, got = _zero_pool_like(h.target_pool), _zero_pool_like(h.target_pool)
        src = pool_rows(h.source_pool, index=h.source_slots)
        plan.launch_batch(src, pool_rows(want, block_table=bt, page_size=16), spans)
        tgt = pool_rows(got, block_table=bt, page_size=16)
        arr = _span_array(spans)
        _lib.check(lib.cb_map_install_batch_noalloc(plan._handle, ctypes.byref(src.c),
                                                    ctypes.byref(tgt.c), arr, len(spans),
                                                    _lib.stream_handle(stream)))
        torch.cuda.synchronize()
        assert plan.read_errors() == 0
        assert torch.equal(got.k_data, want.k_data)
        assert torch.equal(got.v_data, want.v_data)
        assert int(got.v_data.abs().sum()) > 0


def test_noalloc_pooled_batch_equals_allocating_batch():
    """A batch long enough for the streaming kernel's work pool (5,100 tokens
    into the whole 40x8 -> 64x8 model: about 16K weight units per workgroup,
    above the pool threshold of 8,192), then a short one without the pool,
    then the long one again: the pool's claim counters live in plan-owned
    device memory and are cleared by each launch's last workgroup, so the
    no-allocation call needs nothing more."""
    lib = _lib.load()
    batches = [([1500, 2000, 900, 700], [0, 0, 64, 3]), ([300, 1200], [0, 9]),
               ([1500, 2000, 900, 700], [0, 0, 64, 3])]
    tokens = sum(batches[0][0])
    sh = synthetic.shape("full", tokens=tokens)
    pages = sum((n + 15) // 16 for n in batches[0][0]) * 2
    h = synthetic.make_handoff(sh, target_pages=pages, fill_target="zeros", device_source=True)
    plan = h.mapper.plan
    stream = torch.cuda.current_stream()
    for call, (lengths, positions) in enumerate(batches):
        print(f"no-alloc pooled call {call}: {len(lengths)} requests, {sum(lengths)} tokens", flush=True)
        spans, bt = _spans(lengths, positions, pages, seed=40 + call)
        bt = bt.to(h.target_pool.device)
        want, got = _zero_pool_like(h.target_pool), _zero_pool_like(h.target_pool)
        src = pool_rows(h.source_pool, index=h.source_slots)
        plan.launch_batch(src, pool_rows(want, block_table=bt, page_size=16), spans)
        tgt = pool_rows(got, block_table=bt, page_size=16)
        arr = _span_array(spans)
        _lib.check(lib.cb_map_install_batch_noalloc(plan._handle, ctypes.byref(src.c),
                                                    ctypes.byref(tgt.c), arr, len(spans),
                                                    _lib.stream_handle(stream)))
        torch.cuda.synchronize()
        assert plan.read_errors() == 0
        assert torch.equal(got.k_data, want.k_data)
        assert torch.equal(got.v_data, want.v_data)
        assert int(got.v_data.abs().sum()) > 0
        del want, got


def test_noalloc_pooled_batch_replays_from_a_hip_graph():
    """The no-allocation call recorded into a HIP graph (torch.cuda.graph) on
    a batch long enough for the work pool, replayed four times with eager
    launches of the same plan on another stream and host synchronizations in
    between: every replay writes exactly the rows of a direct launch, and the
    error word stays clear. A captured launch takes a counter pair of its own,
    which the direct launches never rotate onto."""
    lib = _lib.load()
    lengths, positions = [1500, 2000, 900, 700], [0, 0, 64, 3]
    tokens = sum(lengths)
    sh = synthetic.shape("full", tokens=tokens)
    pages = sum((n + 15) // 16 for n in lengths) * 2
    h = synthetic.make_handoff(sh, target_pages=pages, fill_target="zeros", device_source=True)
    plan = h.mapper.plan
    spans, bt = _spans(lengths, positions, pages, seed=60)
    bt = bt.to(h.target_pool.device)
    src = pool_rows(h.source_pool, index=h.source_slots)
    want = _zero_pool_like(h.target_pool)
    print(f"graph replay: {len(lengths)} requests, {tokens} tokens, whole model", flush=True)
    plan.launch_batch(src, pool_rows(want, block_table=bt, page_size=16), spans)
    torch.cuda.synchronize()
    assert plan.last_split()[0] > 0, "the batch must be long enough for the work pool"
    assert plan.read_errors() == 0

    got = _zero_pool_like(h.target_pool)
    tgt = pool_rows(got, block_table=bt, page_size=16)
    arr = _span_array(spans)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    other = _zero_pool_like(h.target_pool)
    other_rows = pool_rows(other, block_table=bt, page_size=16)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        _lib.check(lib.cb_map_install_batch_noalloc(plan._handle, ctypes.byref(src.c),
                                                    ctypes.byref(tgt.c), arr, len(spans),
                                                    _lib.stream_handle(torch.cuda.current_stream())))
    for replay in range(4):
        got.k_data.zero_()
        got.v_data.zero_()
        torch.cuda.synchronize()
        graph.replay()
        with torch.cuda.stream(side):
            plan.launch_batch(src, other_rows, spans)
        torch.cuda.synchronize()
        print(f"replay {replay}", flush=True)
        assert plan.read_errors() == 0
        assert torch.equal(got.k_data, want.k_data)
        assert torch.equal(got.v_data, want.v_data)
        assert torch.equal(other.k_data, want.k_data)
    del graph


def test_noalloc_batch_beyond_the_workspace_is_rejected_before_launch():
    lib = _lib.load()
    sh = synthetic.shape("tp4", tokens=64)
    sh.target_layers = 2
    h = synthetic.make_handoff(sh, target_pages=16, fill_target="zeros")
    per = 40000
    count = _lib.CB_NOALLOC_MAX_TOKENS // per + 1
    spans = [RequestSpan(0, 0, per, 0, 0)] * count
    src = pool_rows(h.source_pool, index=h.source_slots)
    tgt = pool_rows(h.target_pool, block_table=h.block_table, page_size=16)
    arr = _span_array(spans)
    with pytest.raises(ValueError, match="no-allocation"):
        _lib.check(lib.cb_map_install_batch_noalloc(h.mapper.plan._handle, ctypes.byref(src.c),
                                                    ctypes.byref(tgt.c), arr, len(spans),
                                                    _lib.stream_handle(None)))
    torch.cuda.synchronize()
    assert int(h.target_pool.k_data.abs().sum()) == 0
