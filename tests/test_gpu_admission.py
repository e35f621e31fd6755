"""GPU: an admitted cohort driven through the admission state machine.

``execute_cohort`` runs one synchronous map+install per request (FIFO);
``execute_cohort_batched`` maps the whole cohort in one launch and then
publishes FIFO. Both must leave identical target pools (bit for bit), publish
in admission order, and dispatch the queries once, after every prefix.
The per-request path is pinned against the oracle by the fused-install parity
tests.
"""

from __future__ import annotations

import pytest
import torch

from cachebridge_amd import synthetic
from cachebridge_amd.online.admission import MapperRequest, OnlineMapperAdmission
from cachebridge_amd.online.blocks import map_install_batch, map_install_block
from cachebridge_amd.pool import PagedKVPool

pytestmark = pytest.mark.gpu


def _empty_like(pool):
    return PagedKVPool(layer_num=pool.layer_num, pages=pool.pages, head_num=pool.head_num,
                       head_dim=pool.head_dim, page_size=pool.page_size, dtype=pool.dtype,
                       device=pool.device, fill="zeros")


def test_batched_cohort_installs_what_serial_cohort_installs():
    lengths = [300, 17, 1024, 64]
    print(f"admission cohort tp4 layers=6 lengths={lengths}", flush=True)
    sh = synthetic.shape("tp4", tokens=sum(lengths))
    sh.target_layers = 6
    bh = synthetic.make_batch_handoff(sh, lengths, occupancy=0.5)
    ps = sh.page_size
    cohort = [MapperRequest(f"req{i}", n) for i, n in enumerate(lengths)]
    span = {r.request_id: sp for r, sp in zip(cohort, bh.spans)}
    available = sum(lengths) + 32 * len(lengths)

    serial_pool, batched_pool = _empty_like(bh.target_pool), _empty_like(bh.target_pool)
    log = []

    def transaction(request):
        sp = span[request.request_id]
        e = sp.target_offset // ps
        map_install_block(bh.mapper, bh.source_pool,
                          bh.source_slots[sp.source_offset:sp.source_offset + sp.num_tokens],
                          serial_pool, start=0, stop=sp.num_tokens,
                          block_table=bh.block_table[e:e + (sp.num_tokens + ps - 1) // ps],
                          page_size=ps)
        torch.cuda.synchronize()
        if bh.mapper.plan.read_errors():
            raise RuntimeError("install flagged rows outside a pool")
        log.append(("serial", request.request_id))

    adm = OnlineMapperAdmission()
    assert adm.execute_cohort(adm.plan(cohort, available_target_tokens=available),
                              mapper_transaction=transaction, query_batch=lambda ids: ids) == \
        tuple(r.request_id for r in cohort)

    def map_cohort(requests):
        map_install_batch(bh.mapper, bh.source_pool, bh.source_slots, batched_pool,
                          [span[r.request_id] for r in requests], block_table=bh.block_table,
                          page_size=ps)
        torch.cuda.synchronize()
        log.append(("batch", len(requests)))

    def publish(request):
        if bh.mapper.plan.read_errors():
            raise RuntimeError("install flagged rows outside a pool")
        log.append(("publish", request.request_id))

    ids = adm.execute_cohort_batched(adm.plan(cohort, available_target_tokens=available),
                                     map_cohort=map_cohort, publish=publish,
                                     query_batch=lambda ids: ids)
    assert ids == tuple(r.request_id for r in cohort)
    assert log[len(cohort):] == [("batch", len(cohort))] + [("publish", r.request_id) for r in cohort]
    assert adm.snapshot()["state"] == "idle"
    assert torch.equal(serial_pool.k_data, batched_pool.k_data)
    assert torch.equal(serial_pool.v_data, batched_pool.v_data)
    for sp in bh.spans:  # every request's first page was written
        row = int(bh.block_table[sp.target_offset // ps]) * ps
        assert batched_pool.v_data[:, row].abs().sum() > 0


def test_batched_cohort_quarantines_when_a_vote_fails_after_the_launch():
    lengths = [40, 56]
    sh = synthetic.shape("tp4", tokens=sum(lengths))
    sh.target_layers = 2
    bh = synthetic.make_batch_handoff(sh, lengths, occupancy=0.5)
    pool = _empty_like(bh.target_pool)
    cohort = [MapperRequest("a", 40), MapperRequest("b", 56)]
    adm = OnlineMapperAdmission(query_reserve_tokens_per_request=0)
    queried = []

    def map_cohort(requests):
        map_install_batch(bh.mapper, bh.source_pool, bh.source_slots, pool, bh.spans,
                          block_table=bh.block_table, page_size=sh.page_size)
        torch.cuda.synchronize()

    def publish(request):
        if request.request_id == "b":
            raise RuntimeError("TP publication vote failed")

    with pytest.raises(RuntimeError, match="vote failed"):
        adm.execute_cohort_batched(adm.plan(cohort, available_target_tokens=96), map_cohort=map_cohort,
                                   publish=publish, query_batch=queried.append)
    snap = adm.snapshot()
    assert (snap["state"], snap["active_request"], snap["published_request_ids"]) == \
        ("quarantined", "b", ("a",))
    assert queried == []
