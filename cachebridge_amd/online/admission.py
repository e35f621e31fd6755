"""Admission of handoff requests around the GPU map (host logic).

Mirrors the reference's online admission contracts
(``cb/online/admission.py:24-565``; ``cb/`` = ``src/cachebridge/``):

- ``LiveMapperMechanism`` (``:42-82``): the fail-closed capability contract
  that must hold before mapping may overlap target decode;
- ``LiveMapperCostPolicy`` (``:85-104``): the break-even gate on history
  length;
- ``OnlineMapperRouter`` (``:134-253``): live mapper, cohort mapper, native
  re-prefill or backpressure, and dispatch of exactly one path;
- ``LiveMapperAdmission`` (``:256-394``): one unpublished transaction that
  publishes only with GPU completion and the TP vote;
- ``OnlineMapperAdmission`` (``:397-565``): the one-cohort state machine,
  FIFO publication, one coalesced query batch.

One addition: ``OnlineMapperAdmission.execute_cohort_batched`` maps a whole
admitted cohort with one GPU launch (``cb_map_install_batch``, every row
identical to the per-request launches) and then publishes the requests in FIFO
order through the same state machine, where ``execute_cohort`` runs one mapper
transaction per request.
"""

from __future__ import annotations

from collections.abc import Callable, Iterable
from dataclasses import dataclass
from typing import Literal, TypeVar

_Result = TypeVar("_Result")


@dataclass(frozen=True)
class MapperRequest:
    request_id: str
    history_tokens: int


@dataclass(frozen=True)
class AdmissionPlan:
    admitted: bool
    reason: str
    requests: tuple
    required_target_tokens: int
    available_target_tokens: int
    mapper_transactions_in_flight: int
    mapper_workspace_scales_with_cohort: bool
    query_coalescing: bool


@dataclass(frozen=True)
class LiveMapperMechanism:
    """Capabilities that must all hold before mapper work overlaps target decode."""

    mapper_compute_role: Literal["source", "target"] = "source"
    mapped_output_slots: int = 2
    direct_target_placement: bool = True
    target_mapper_workspace_bytes: int = 0
    target_transfer_workspace_bytes: int = 0
    scheduler_serialized_allocation: bool = True
    scheduler_serialized_publication: bool = True
    source_slot_gpu_ack: bool = True
    max_staged_transactions: int = 1

    def validate(self) -> None:
        checks = (
            (self.mapper_compute_role == "source", "live mapper compute must be source-isolated"),
            (self.mapped_output_slots >= 2, "live mapper requires at least two output slots"),
            (self.direct_target_placement, "live mapper requires direct target placement"),
            (self.target_mapper_workspace_bytes == 0, "live mapper cannot allocate target mapper workspace"),
            (self.target_transfer_workspace_bytes == 0, "live mapper cannot allocate target transfer workspace"),
            (self.scheduler_serialized_allocation, "target allocation must be scheduler-serialized"),
            (self.scheduler_serialized_publication, "target publication must be scheduler-serialized"),
            (self.source_slot_gpu_ack, "source slots require target GPU-complete ACKs"),
            (self.max_staged_transactions == 1, "exactly one unpublished transaction is supported"),
        )
        for ok, message in checks:
            if not ok:
                raise ValueError(message)


@dataclass(frozen=True)
class LiveMapperCostPolicy:
    """Map a request live only when its history is long enough to pay off."""

    min_history_tokens: int
    objective: Literal["ttft"] = "ttft"

    def validate(self) -> None:
        if self.min_history_tokens <= 0:
            raise ValueError("min_history_tokens must be positive")
        if self.objective != "ttft":
            raise ValueError("only the measured ttft objective is supported")

    def admits(self, request: MapperRequest) -> bool:
        return request.history_tokens >= self.min_history_tokens


@dataclass(frozen=True)
class LiveAdmissionPlan:
    admitted: bool
    reason: str
    request: MapperRequest
    required_target_tokens: int
    available_target_tokens: int
    decoder_active: bool


@dataclass(frozen=True)
class PublicationProof:
    gpu_reads_complete: bool
    tp_vote_passed: bool


@dataclass(frozen=True)
class RouterDecision:
    mode: Literal["cachebridge_live", "cachebridge_cohort", "native_reprefill", "backpressure"]
    reason: str
    requests: tuple
    canceled_request_ids: tuple
    decoder_active: bool
    service_class: Literal["latency", "throughput"]
    cohort_preformed: bool


def _check_identities(ids) -> None:
    if any(not i for i in ids):
        raise ValueError("request identity must be non-empty")
    if len(set(ids)) != len(ids):
        raise ValueError("request identities must be unique")


class OnlineMapperRouter:
    """Choose the serving path of an arrival cohort."""

    def __init__(self, *, max_cohort_requests: int = 4, live_mechanism: LiveMapperMechanism | None = None,
                 live_cost_policy: LiveMapperCostPolicy | None = None) -> None:
        if max_cohort_requests <= 0:
            raise ValueError("max_cohort_requests must be positive")
        if live_mechanism is not None:
            live_mechanism.validate()
        if live_cost_policy is not None:
            live_cost_policy.validate()
            if live_mechanism is None:
                raise ValueError("live cost policy requires a live mapper mechanism")
        self.max_cohort_requests = max_cohort_requests
        self.live_mechanism = live_mechanism
        self.live_cost_policy = live_cost_policy

    def route(self, requests: Iterable[MapperRequest], *, decoder_active: bool,
              service_class: Literal["latency", "throughput"], cohort_preformed: bool,
              canceled_request_ids: Iterable[str] = ()) -> RouterDecision:
        cohort = tuple(requests)
        if not cohort:
            raise ValueError("route requires at least one request")
        ids = [r.request_id for r in cohort]
        _check_identities(ids)
        canceled = tuple(canceled_request_ids)
        if len(set(canceled)) != len(canceled):
            raise ValueError("canceled request identities must be unique")
        unknown = set(canceled) - set(ids)
        if unknown:
            raise ValueError(f"unknown canceled request identities: {sorted(unknown)}")
        active = tuple(r for r in cohort if r.request_id not in set(canceled))

        def decide(mode, reason, reqs=active):
            return RouterDecision(mode, reason, reqs, canceled, decoder_active, service_class, cohort_preformed)

        if not active:
            return decide("backpressure", "cohort_canceled", ())
        if len(active) > self.max_cohort_requests:
            return decide("backpressure", "cohort_request_limit")
        if self.live_mechanism is not None:
            if self.live_cost_policy is not None and not all(self.live_cost_policy.admits(r) for r in active):
                return decide("native_reprefill", "below_live_mapper_break_even")
            return decide("cachebridge_live", "source_isolated_live_mapper")
        if decoder_active:
            return decide("native_reprefill", "decoder_active")
        if service_class == "latency":
            return decide("native_reprefill", "latency_service_class")
        if not cohort_preformed:
            return decide("native_reprefill", "trickle_arrival_no_wait")
        return decide("cachebridge_cohort", "idle_preformed_throughput_cohort")

    def dispatch(self, decision: RouterDecision, *, cachebridge_live: Callable | None = None,
                 cachebridge_cohort: Callable, native_reprefill: Callable):
        """Run exactly the one serving path the decision selected."""
        if decision.mode == "cachebridge_live":
            if cachebridge_live is None:
                raise RuntimeError("cachebridge_live callback is required")
            return cachebridge_live(decision.requests)
        if decision.mode == "cachebridge_cohort":
            return cachebridge_cohort(decision.requests)
        if decision.mode == "native_reprefill":
            return native_reprefill(decision.requests)
        raise RuntimeError(f"cannot dispatch backpressured route: {decision.reason}")


class LiveMapperAdmission:
    """One unpublished post-arrival mapper transaction at a time."""

    def __init__(self, *, mechanism: LiveMapperMechanism, query_reserve_tokens: int = 32) -> None:
        if query_reserve_tokens < 0:
            raise ValueError("query reserve must be non-negative")
        mechanism.validate()
        self.mechanism = mechanism
        self.query_reserve_tokens = query_reserve_tokens
        self._active: MapperRequest | None = None
        self._phase = "idle"
        self._decoder_active = False
        self._completed: list[str] = []
        self._error: str | None = None

    def plan(self, request: MapperRequest, *, available_target_tokens: int,
             decoder_active: bool) -> LiveAdmissionPlan:
        if not request.request_id:
            raise ValueError("request identity must be non-empty")
        if request.history_tokens <= 0:
            raise ValueError("history_tokens must be positive")
        required = request.history_tokens + self.query_reserve_tokens
        if self._phase != "idle":
            admitted, reason = False, "mapper_transaction_in_flight"
        elif required > available_target_tokens:
            admitted, reason = False, "target_token_backpressure"
        else:
            admitted, reason = True, "admitted_during_decode" if decoder_active else "admitted"
        return LiveAdmissionPlan(admitted, reason, request, required, available_target_tokens, decoder_active)

    def begin(self, plan: LiveAdmissionPlan) -> MapperRequest:
        if self._phase != "idle":
            raise RuntimeError(f"cannot begin while state={self._phase}")
        if not plan.admitted:
            raise RuntimeError(f"cannot execute rejected plan: {plan.reason}")
        if plan.request.request_id in self._completed:
            raise RuntimeError("request identity was already published")
        self._active, self._decoder_active = plan.request, plan.decoder_active
        self._phase, self._error = "mapping", None
        return plan.request

    def mark_source_complete(self, request_id: str) -> None:
        self._own(request_id, "mapping")
        self._phase = "source_ready"

    def publish(self, request_id: str, proof: PublicationProof) -> None:
        self._own(request_id, "source_ready")
        if not (proof.gpu_reads_complete and proof.tp_vote_passed):
            self.quarantine("publication proof failed")
            raise RuntimeError("cannot publish without GPU completion and TP vote")
        self._phase = "published"

    def mark_submitted(self, request_id: str) -> None:
        self._own(request_id, "published")
        self._completed.append(request_id)
        self._active, self._decoder_active, self._phase = None, False, "idle"

    def rollback(self, request_id: str, *, gpu_reads_complete: bool, target_pages_released: bool) -> None:
        if self._active is None or self._active.request_id != request_id:
            raise RuntimeError("rollback does not own the active transaction")
        if self._phase not in ("mapping", "source_ready"):
            raise RuntimeError(f"cannot roll back while state={self._phase}")
        if not (gpu_reads_complete and target_pages_released):
            self.quarantine("unsafe rollback")
            raise RuntimeError("rollback requires completed reads and released pages")
        self._active, self._decoder_active, self._phase = None, False, "idle"

    def quarantine(self, error) -> None:
        self._phase, self._error = "quarantined", str(error)

    def snapshot(self) -> dict:
        m = self.mechanism
        return {
            "state": self._phase,
            "active_request": None if self._active is None else self._active.request_id,
            "decoder_active_during_mapping": self._decoder_active,
            "completed_request_ids": tuple(self._completed),
            "error": self._error,
            "mapper_compute_role": m.mapper_compute_role,
            "mapped_output_slots": m.mapped_output_slots,
            "max_staged_transactions": m.max_staged_transactions,
            "target_mapper_workspace_bytes": m.target_mapper_workspace_bytes,
            "target_transfer_workspace_bytes": m.target_transfer_workspace_bytes,
            "direct_target_placement": m.direct_target_placement,
            "scheduler_serialized_publication": m.scheduler_serialized_publication,
        }

    def _own(self, request_id: str, phase: str) -> None:
        if self._phase != phase or self._active is None or self._active.request_id != request_id:
            raise RuntimeError("operation does not own the active mapper transaction")


class OnlineMapperAdmission:
    """One admitted cohort: FIFO mapper transactions, then one query batch."""

    def __init__(self, *, max_cohort_requests: int = 4, query_reserve_tokens_per_request: int = 32) -> None:
        if max_cohort_requests <= 0:
            raise ValueError("max_cohort_requests must be positive")
        if query_reserve_tokens_per_request < 0:
            raise ValueError("query reserve must be non-negative")
        self.max_cohort_requests = max_cohort_requests
        self.query_reserve_tokens_per_request = query_reserve_tokens_per_request
        self._reset("idle")

    def _reset(self, state: str) -> None:
        self._state = state
        self._requests: tuple = ()
        self._pending: list[str] = []
        self._published: list[str] = []
        self._active_request: str | None = None
        self._error: str | None = None

    def plan(self, requests: Iterable[MapperRequest], *, available_target_tokens: int) -> AdmissionPlan:
        cohort = tuple(requests)
        if not cohort:
            raise ValueError("cohort must be non-empty")
        if len(cohort) > self.max_cohort_requests:
            return AdmissionPlan(False, "cohort_request_limit", cohort, 0, available_target_tokens, 0, False, True)
        _check_identities([r.request_id for r in cohort])
        if any(r.history_tokens <= 0 for r in cohort):
            raise ValueError("history_tokens must be positive")
        required = sum(r.history_tokens for r in cohort) + len(cohort) * self.query_reserve_tokens_per_request
        admitted = required <= available_target_tokens
        return AdmissionPlan(admitted, "admitted" if admitted else "target_token_backpressure", cohort, required,
                             available_target_tokens, 1 if admitted else 0, False, True)

    def admit(self, plan: AdmissionPlan) -> None:
        if self._state != "idle":
            raise RuntimeError(f"cannot admit while state={self._state}")
        if not plan.admitted:
            raise RuntimeError(f"cannot execute rejected plan: {plan.reason}")
        self._reset("admitted")
        self._requests = plan.requests
        self._pending = [r.request_id for r in plan.requests]

    def begin_next_mapper(self) -> MapperRequest:
        if self._state not in ("admitted", "mapping"):
            raise RuntimeError(f"cannot start mapper while state={self._state}")
        if self._active_request is not None:
            raise RuntimeError("another mapper transaction is active")
        if not self._pending:
            raise RuntimeError("cohort has no pending mapper request")
        self._active_request = self._pending[0]
        self._state = "mapping"
        return next(r for r in self._requests if r.request_id == self._active_request)

    def publish_active_mapper(self, request_id: str) -> None:
        if self._state != "mapping" or self._active_request != request_id:
            raise RuntimeError("publication does not own the active mapper transaction")
        if not self._pending or self._pending[0] != request_id:
            raise RuntimeError("mapper completion violated FIFO admission order")
        self._published.append(self._pending.pop(0))
        self._active_request = None
        self._state = "mapping" if self._pending else "ready"

    def coalesced_query_batch(self) -> tuple:
        if self._state != "ready" or self._active_request is not None or self._pending:
            raise RuntimeError("queries cannot dispatch before every prefix is published")
        expected = tuple(r.request_id for r in self._requests)
        if tuple(self._published) != expected:
            raise RuntimeError("published request set differs from admitted cohort")
        self._state = "dispatched"
        return expected

    def finish_queries(self) -> None:
        if self._state != "dispatched":
            raise RuntimeError(f"cannot finish queries while state={self._state}")
        self._reset("idle")

    def execute_cohort(self, plan: AdmissionPlan, *, mapper_transaction: Callable[[MapperRequest], None],
                       query_batch: Callable[[tuple], _Result]) -> _Result:
        """One synchronous mapper transaction per request (map, install, checks
        and the TP vote inside the callback), then one query batch. A callback
        failure quarantines the cohort and is re-raised."""
        self.admit(plan)
        try:
            while self._pending:
                request = self.begin_next_mapper()
                mapper_transaction(request)
                self.publish_active_mapper(request.request_id)
            result = query_batch(self.coalesced_query_batch())
        except BaseException as error:
            self.quarantine(error)
            raise
        self.finish_queries()
        return result

    def execute_cohort_batched(self, plan: AdmissionPlan, *, map_cohort: Callable[[tuple], None],
                               publish: Callable[[MapperRequest], None],
                               query_batch: Callable[[tuple], _Result]) -> _Result:
        """Map every admitted request in one launch, then publish in FIFO order.

        ``map_cohort(requests)`` must return after the cohort's map and install
        have completed on the GPU (e.g. ``map_install_batch`` followed by a
        stream synchronization). ``publish(request)`` runs each request's safety
        checks and TP vote, in admission order; a failure quarantines the
        cohort with that request active and is re-raised.
        """
        self.admit(plan)
        try:
            map_cohort(self._requests)
            while self._pending:
                request = self.begin_next_mapper()
                publish(request)
                self.publish_active_mapper(request.request_id)
            result = query_batch(self.coalesced_query_batch())
        except BaseException as error:
            self.quarantine(error)
            raise
        self.finish_queries()
        return result

    def quarantine(self, error) -> None:
        self._state, self._error = "quarantined", str(error)

    def snapshot(self) -> dict:
        return {
            "state": self._state,
            "active_request": self._active_request,
            "pending_request_ids": tuple(self._pending),
            "published_request_ids": tuple(self._published),
            "error": self._error,
            "max_mapper_transactions_in_flight": 1,
            "mapper_workspace_scales_with_cohort": False,
            "query_coalescing": True,
        }

