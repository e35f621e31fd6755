"""Admission host logic: the reference's contracts (``tests/test_admission.py``
of the reference, all 19 cases restated) plus the one-launch cohort path.

Host state machines only; nothing here touches a GPU.
"""

from __future__ import annotations

import dataclasses

import pytest

from cachebridge_amd.online.admission import (
    LiveMapperAdmission,
    LiveMapperCostPolicy,
    LiveMapperMechanism,
    MapperRequest,
    OnlineMapperAdmission,
    OnlineMapperRouter,
    PublicationProof,
)


def requests(*history):
    return [MapperRequest(f"r{i}", n) for i, n in enumerate(history)]


def noop(_):
    return None


# --- OnlineMapperAdmission (cohort state machine) ---------------------------------------------


def test_capacity_rejects_without_partial_state():
    adm = OnlineMapperAdmission(query_reserve_tokens_per_request=4)
    plan = adm.plan(requests(100, 200), available_target_tokens=307)
    assert (plan.admitted, plan.reason, plan.required_target_tokens) == \
        (False, "target_token_backpressure", 308)
    assert plan.mapper_transactions_in_flight == 0
    assert adm.snapshot()["state"] == "idle"
    # one token more admits, with exactly one transaction in flight
    ok = adm.plan(requests(100, 200), available_target_tokens=308)
    assert ok.admitted and ok.mapper_transactions_in_flight == 1
    assert not ok.mapper_workspace_scales_with_cohort and ok.query_coalescing


def test_mapper_is_fifo_serial_and_queries_coalesce_after_publication():
    adm = OnlineMapperAdmission(query_reserve_tokens_per_request=0)
    adm.admit(adm.plan(requests(8, 8, 8), available_target_tokens=24))
    assert adm.begin_next_mapper().request_id == "r0"
    with pytest.raises(RuntimeError, match="another mapper transaction"):
        adm.begin_next_mapper()
    adm.publish_active_mapper("r0")
    with pytest.raises(RuntimeError, match="every prefix"):
        adm.coalesced_query_batch()
    for rid in ("r1", "r2"):
        assert adm.begin_next_mapper().request_id == rid
        adm.publish_active_mapper(rid)
    assert adm.coalesced_query_batch() == ("r0", "r1", "r2")
    adm.finish_queries()
    snap = adm.snapshot()
    assert snap["state"] == "idle" and snap["published_request_ids"] == ()


def test_identity_and_ownership_mismatch_fail_closed():
    adm = OnlineMapperAdmission(query_reserve_tokens_per_request=0)
    with pytest.raises(ValueError, match="unique"):
        adm.plan([MapperRequest("dup", 8), MapperRequest("dup", 8)], available_target_tokens=16)
    with pytest.raises(ValueError, match="non-empty"):
        adm.plan([MapperRequest("", 8)], available_target_tokens=16)
    with pytest.raises(ValueError, match="positive"):
        adm.plan([MapperRequest("a", 0)], available_target_tokens=16)
    adm.admit(adm.plan(requests(8), available_target_tokens=8))
    adm.begin_next_mapper()
    with pytest.raises(RuntimeError, match="does not own"):
        adm.publish_active_mapper("someone-else")
    adm.quarantine("ownership mismatch")
    snap = adm.snapshot()
    assert snap["state"] == "quarantined" and snap["error"] == "ownership mismatch"
    with pytest.raises(RuntimeError, match="state=quarantined"):
        adm.admit(adm.plan(requests(8), available_target_tokens=8))


def test_execute_cohort_connects_serial_mapper_to_one_query_batch():
    adm = OnlineMapperAdmission(query_reserve_tokens_per_request=0)
    plan = adm.plan(requests(8, 12, 16), available_target_tokens=36)
    log = []

    def query_batch(ids):
        log.append(("queries", ids))
        return dict.fromkeys(ids, "tok")

    out = adm.execute_cohort(plan, mapper_transaction=lambda r: log.append(("map", r.request_id)),
                             query_batch=query_batch)
    assert log == [("map", "r0"), ("map", "r1"), ("map", "r2"), ("queries", ("r0", "r1", "r2"))]
    assert out == {"r0": "tok", "r1": "tok", "r2": "tok"}
    assert adm.snapshot()["state"] == "idle"


def test_execute_cohort_quarantines_callback_failure():
    adm = OnlineMapperAdmission(query_reserve_tokens_per_request=0)
    plan = adm.plan(requests(8, 8), available_target_tokens=16)

    def transaction(r):
        if r.request_id == "r1":
            raise OSError("TP publication vote failed")

    with pytest.raises(OSError, match="publication vote"):
        adm.execute_cohort(plan, mapper_transaction=transaction, query_batch=lambda ids: ids)
    snap = adm.snapshot()
    assert (snap["state"], snap["active_request"], snap["error"]) == \
        ("quarantined", "r1", "TP publication vote failed")
    assert snap["published_request_ids"] == ("r0",)


def test_rejected_or_oversized_plan_cannot_be_admitted():
    adm = OnlineMapperAdmission(max_cohort_requests=2, query_reserve_tokens_per_request=0)
    big = adm.plan(requests(1, 1, 1), available_target_tokens=100)
    assert (big.admitted, big.reason, big.required_target_tokens) == (False, "cohort_request_limit", 0)
    with pytest.raises(RuntimeError, match="cohort_request_limit"):
        adm.admit(big)
    with pytest.raises(ValueError, match="non-empty"):
        adm.plan([], available_target_tokens=1)
    with pytest.raises(ValueError, match="max_cohort_requests"):
        OnlineMapperAdmission(max_cohort_requests=0)
    with pytest.raises(ValueError, match="non-negative"):
        OnlineMapperAdmission(query_reserve_tokens_per_request=-1)


# --- one-launch cohort: map everything, then publish FIFO ------------------------------------


def test_batched_cohort_maps_once_then_publishes_fifo():
    adm = OnlineMapperAdmission(query_reserve_tokens_per_request=2)
    plan = adm.plan(requests(8, 12, 16), available_target_tokens=42)
    log = []
    out = adm.execute_cohort_batched(
        plan,
        map_cohort=lambda rs: log.append(("map", tuple(r.request_id for r in rs))),
        publish=lambda r: log.append(("publish", r.request_id, adm.snapshot()["active_request"])),
        query_batch=lambda ids: log.append(("queries", ids)) or len(ids))
    assert log == [("map", ("r0", "r1", "r2")), ("publish", "r0", "r0"), ("publish", "r1", "r1"),
                   ("publish", "r2", "r2"), ("queries", ("r0", "r1", "r2"))]
    assert out == 3 and adm.snapshot()["state"] == "idle"


def test_batched_cohort_quarantines_map_or_vote_failure():
    adm = OnlineMapperAdmission(query_reserve_tokens_per_request=0)
    plan = adm.plan(requests(8, 8), available_target_tokens=16)

    def bad_map(_):
        raise RuntimeError("map launch failed")

    with pytest.raises(RuntimeError, match="map launch failed"):
        adm.execute_cohort_batched(plan, map_cohort=bad_map, publish=noop, query_batch=noop)
    snap = adm.snapshot()
    assert snap["state"] == "quarantined" and snap["published_request_ids"] == ()
    assert snap["pending_request_ids"] == ("r0", "r1")

    adm2 = OnlineMapperAdmission(query_reserve_tokens_per_request=0)
    queried = []

    def vote(r):
        if r.request_id == "r1":
            raise OSError("TP publication vote failed")

    with pytest.raises(OSError):
        adm2.execute_cohort_batched(adm2.plan(requests(8, 8), available_target_tokens=16),
                                    map_cohort=noop, publish=vote, query_batch=queried.append)
    snap = adm2.snapshot()
    assert (snap["state"], snap["active_request"], snap["published_request_ids"]) == \
        ("quarantined", "r1", ("r0",))
    assert queried == []  # no query runs before every prefix is published


# --- OnlineMapperRouter -----------------------------------------------------------------------


def route(router, reqs, *, decoder_active=False, service_class="throughput", cohort_preformed=True,
          canceled=()):
    return router.route(reqs, decoder_active=decoder_active, service_class=service_class,
                        cohort_preformed=cohort_preformed, canceled_request_ids=canceled)


def test_router_uses_cachebridge_only_for_idle_preformed_throughput_cohort():
    d = route(OnlineMapperRouter(), requests(8, 8))
    assert (d.mode, d.reason) == ("cachebridge_cohort", "idle_preformed_throughput_cohort")
    assert [r.request_id for r in d.requests] == ["r0", "r1"]


@pytest.mark.parametrize("decoder_active,service_class,cohort_preformed", [
    (True, "throughput", True), (True, "latency", False), (False, "latency", False)])
def test_source_isolated_live_mapper_handles_decoder_active_and_trickle_arrivals(
        decoder_active, service_class, cohort_preformed):
    router = OnlineMapperRouter(live_mechanism=LiveMapperMechanism())
    d = route(router, requests(8), decoder_active=decoder_active, service_class=service_class,
              cohort_preformed=cohort_preformed)
    assert (d.mode, d.reason) == ("cachebridge_live", "source_isolated_live_mapper")
    called = []
    out = router.dispatch(d, cachebridge_live=lambda rs: called.append("live") or "done",
                          cachebridge_cohort=lambda rs: called.append("cohort"),
                          native_reprefill=lambda rs: called.append("native"))
    assert out == "done" and called == ["live"]
    with pytest.raises(RuntimeError, match="cachebridge_live callback"):
        router.dispatch(d, cachebridge_cohort=noop, native_reprefill=noop)


@pytest.mark.parametrize("decoder_active", [False, True])
def test_live_cost_policy_routes_below_break_even_to_native_without_idle_wait(decoder_active):
    router = OnlineMapperRouter(live_mechanism=LiveMapperMechanism(),
                                live_cost_policy=LiveMapperCostPolicy(min_history_tokens=4096))
    short = route(router, requests(4095), decoder_active=decoder_active, service_class="latency",
                  cohort_preformed=False)
    assert (short.mode, short.reason) == ("native_reprefill", "below_live_mapper_break_even")
    edge = route(router, requests(4096), decoder_active=decoder_active, service_class="latency",
                 cohort_preformed=False)
    assert (edge.mode, edge.reason) == ("cachebridge_live", "source_isolated_live_mapper")


def test_live_cost_policy_routes_an_atomic_mixed_cohort_to_native():
    router = OnlineMapperRouter(live_mechanism=LiveMapperMechanism(),
                                live_cost_policy=LiveMapperCostPolicy(min_history_tokens=4096))
    d = route(router, requests(8192, 2048), decoder_active=True)
    assert (d.mode, d.reason) == ("native_reprefill", "below_live_mapper_break_even")
    assert len(d.requests) == 2  # the cohort is not split


@pytest.mark.parametrize("threshold", [0, -1])
def test_live_cost_policy_rejects_invalid_threshold(threshold):
    with pytest.raises(ValueError, match="min_history_tokens"):
        OnlineMapperRouter(live_mechanism=LiveMapperMechanism(),
                           live_cost_policy=LiveMapperCostPolicy(min_history_tokens=threshold))


def test_live_cost_policy_rejects_unmeasured_objective():
    with pytest.raises(ValueError, match="ttft"):
        LiveMapperCostPolicy(min_history_tokens=1, objective="throughput").validate()


def test_live_cost_policy_requires_live_mechanism():
    with pytest.raises(ValueError, match="requires a live mapper mechanism"):
        OnlineMapperRouter(live_cost_policy=LiveMapperCostPolicy(min_history_tokens=4096))


@pytest.mark.parametrize("field,value,message", [
    ("mapper_compute_role", "target", "source-isolated"),
    ("mapped_output_slots", 1, "two output slots"),
    ("direct_target_placement", False, "direct target placement"),
    ("target_mapper_workspace_bytes", 1, "target mapper workspace"),
    ("target_transfer_workspace_bytes", 1, "target transfer workspace"),
    ("scheduler_serialized_allocation", False, "allocation"),
    ("scheduler_serialized_publication", False, "publication"),
    ("source_slot_gpu_ack", False, "GPU-complete ACKs"),
    ("max_staged_transactions", 2, "one unpublished transaction"),
])
def test_live_mechanism_fails_closed_when_an_isolation_property_is_missing(field, value, message):
    broken = dataclasses.replace(LiveMapperMechanism(), **{field: value})
    with pytest.raises(ValueError, match=message):
        OnlineMapperRouter(live_mechanism=broken)
    with pytest.raises(ValueError, match=message):
        LiveMapperAdmission(mechanism=broken)


@pytest.mark.parametrize("decoder_active,service_class,cohort_preformed,reason", [
    (True, "throughput", True, "decoder_active"),
    (False, "latency", True, "latency_service_class"),
    (False, "throughput", False, "trickle_arrival_no_wait"),
])
def test_router_falls_back_to_native_without_waiting(decoder_active, service_class,
                                                      cohort_preformed, reason):
    d = route(OnlineMapperRouter(), requests(8), decoder_active=decoder_active,
              service_class=service_class, cohort_preformed=cohort_preformed)
    assert (d.mode, d.reason) == ("native_reprefill", reason)


def test_router_removes_canceled_request_before_dispatch():
    router = OnlineMapperRouter()
    d = route(router, requests(8, 8, 8), decoder_active=True, canceled=["r1"])
    called = []
    out = router.dispatch(d, cachebridge_cohort=lambda rs: called.append(("cohort", rs)),
                          native_reprefill=lambda rs: called.append(("native", rs)) or "ok")
    assert out == "ok"
    assert d.canceled_request_ids == ("r1",)
    assert [(name, tuple(r.request_id for r in rs)) for name, rs in called] == \
        [("native", ("r0", "r2"))]


def test_router_rejects_bad_identities_and_cancellations():
    router = OnlineMapperRouter()
    with pytest.raises(ValueError, match="at least one"):
        route(router, [])
    with pytest.raises(ValueError, match="unique"):
        route(router, [MapperRequest("a", 1), MapperRequest("a", 2)])
    with pytest.raises(ValueError, match="unknown canceled"):
        route(router, requests(8), canceled=["zz"])
    with pytest.raises(ValueError, match="canceled request identities must be unique"):
        route(router, requests(8), canceled=["r0", "r0"])
    d = route(router, requests(8, 8), canceled=["r0", "r1"])
    assert (d.mode, d.reason, d.requests) == ("backpressure", "cohort_canceled", ())


def test_router_backpressures_oversized_cohort():
    router = OnlineMapperRouter(max_cohort_requests=2)
    d = route(router, requests(8, 8, 8))
    assert d.mode == "backpressure"
    with pytest.raises(RuntimeError, match="cohort_request_limit"):
        router.dispatch(d, cachebridge_cohort=noop, native_reprefill=noop)
    # cancellation is applied before the limit
    assert route(router, requests(8, 8, 8), canceled=["r2"]).mode == "cachebridge_cohort"


# --- LiveMapperAdmission (one unpublished transaction) ----------------------------------------

OK = PublicationProof(gpu_reads_complete=True, tp_vote_passed=True)


def test_live_admission_publishes_during_active_decode_with_proof():
    adm = LiveMapperAdmission(mechanism=LiveMapperMechanism(), query_reserve_tokens=4)
    req = MapperRequest("late-arrival", 8)
    plan = adm.plan(req, available_target_tokens=12, decoder_active=True)
    assert (plan.admitted, plan.reason, plan.required_target_tokens) == (True, "admitted_during_decode", 12)
    assert not adm.plan(req, available_target_tokens=11, decoder_active=True).admitted
    adm.begin(plan)
    assert adm.snapshot()["decoder_active_during_mapping"]
    adm.mark_source_complete(req.request_id)
    adm.publish(req.request_id, OK)
    adm.mark_submitted(req.request_id)
    snap = adm.snapshot()
    assert snap["state"] == "idle" and snap["completed_request_ids"] == ("late-arrival",)
    assert snap["target_mapper_workspace_bytes"] == 0 and snap["target_transfer_workspace_bytes"] == 0
    # an identity is published once
    with pytest.raises(RuntimeError, match="already published"):
        adm.begin(adm.plan(req, available_target_tokens=12, decoder_active=False))


def test_live_admission_serializes_unpublished_ownership_and_fails_closed():
    adm = LiveMapperAdmission(mechanism=LiveMapperMechanism())
    adm.begin(adm.plan(requests(8)[0], available_target_tokens=40, decoder_active=True))
    second = adm.plan(MapperRequest("second", 8), available_target_tokens=40, decoder_active=True)
    assert (second.admitted, second.reason) == (False, "mapper_transaction_in_flight")
    with pytest.raises(RuntimeError, match="does not own"):
        adm.publish("r0", OK)  # not source-complete yet
    adm.mark_source_complete("r0")
    with pytest.raises(RuntimeError, match="GPU completion and TP vote"):
        adm.publish("r0", PublicationProof(gpu_reads_complete=True, tp_vote_passed=False))
    snap = adm.snapshot()
    assert snap["state"] == "quarantined" and snap["error"] == "publication proof failed"


def test_live_admission_safe_rollback_releases_transaction():
    adm = LiveMapperAdmission(mechanism=LiveMapperMechanism())
    adm.begin(adm.plan(requests(8)[0], available_target_tokens=40, decoder_active=False))
    with pytest.raises(RuntimeError, match="does not own"):
        adm.rollback("other", gpu_reads_complete=True, target_pages_released=True)
    adm.rollback("r0", gpu_reads_complete=True, target_pages_released=True)
    assert adm.snapshot()["state"] == "idle"
    # an unsafe rollback quarantines
    adm.begin(adm.plan(requests(8)[0], available_target_tokens=40, decoder_active=False))
    with pytest.raises(RuntimeError, match="released pages"):
        adm.rollback("r0", gpu_reads_complete=False, target_pages_released=True)
    assert adm.snapshot()["state"] == "quarantined"


def test_live_admission_cannot_roll_back_published_prefix():
    adm = LiveMapperAdmission(mechanism=LiveMapperMechanism())
    adm.begin(adm.plan(requests(8)[0], available_target_tokens=40, decoder_active=True))
    adm.mark_source_complete("r0")
    adm.publish("r0", OK)
    with pytest.raises(RuntimeError, match="state=published"):
        adm.rollback("r0", gpu_reads_complete=True, target_pages_released=True)


def test_batched_cohort_snapshot_reports_its_workspace():
    adm = OnlineMapperAdmission(query_reserve_tokens_per_request=0)
    seen = []
    adm.execute_cohort_batched(adm.plan(requests(8, 12), available_target_tokens=20),
                               map_cohort=lambda rs: seen.append(adm.snapshot()),
                               publish=noop, query_batch=noop)
    assert seen[0]["mapper_workspace_scales_with_cohort"]
    assert seen[0]["mapper_workspace_bytes"] == 12 * 20
    idle = adm.snapshot()  # released with the cohort
    assert not idle["mapper_workspace_scales_with_cohort"] and idle["mapper_workspace_bytes"] == 0
    adm.execute_cohort(adm.plan(requests(8), available_target_tokens=8),
                       mapper_transaction=lambda r: seen.append(adm.snapshot()), query_batch=noop)
    assert seen[1]["mapper_workspace_bytes"] == 0


def test_live_mechanism_lists_every_missing_property():
    broken = dataclasses.replace(LiveMapperMechanism(), mapped_output_slots=1, source_slot_gpu_ack=False)
    assert broken.unmet_requirements() == ["live mapper requires at least two output slots",
                                           "source slots require target GPU-complete ACKs"]
    assert dataclasses.replace(LiveMapperMechanism(), mapped_output_slots=3).unmet_requirements() == []
