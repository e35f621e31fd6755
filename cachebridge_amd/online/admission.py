"""Admission of handoff requests around the GPU map (host logic).

The public contract is the reference's (``cb/online/admission.py:24-565``,
``cb/`` = ``src/cachebridge/``): the same class and dataclass names and
fields, the same reason strings a scheduler routes on, and the same error
texts callers match. The machinery is this module's own:

- every controller is a small table-driven state machine: a method names a
  step, the table says which state the step leaves from and which it enters,
  and ownership of the request being stepped is checked before the move;
- a cohort is a ``_Ledger``: its request ids in admission order and a
  publication cursor (everything before the cursor is published, the request
  at the cursor is the only one that may be mapped), so FIFO order holds by
  construction rather than by bookkeeping of separate lists;
- the router is an ordered list of rules, evaluated first-match;
- the live mapper's isolation properties are compared field by field with
  the one configuration that is allowed (``_ISOLATED``).

``OnlineMapperAdmission.execute_cohort_batched`` is an addition: the whole
admitted cohort is mapped in one launch (``cb_map_install_batch``, every row
identical to the per-request launches), then published request by request in
admission order through the same state machine.
"""

from __future__ import annotations

from collections.abc import Callable, Iterable, Sequence
from dataclasses import dataclass, fields
from typing import Literal, TypeVar

_Result = TypeVar("_Result")

# Bytes of device workspace per mapped token of a one-launch cohort: the
# int32 source row, target row and position the batch resolver writes.
BATCH_WORKSPACE_BYTES_PER_TOKEN = 12


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


def _require_identities(ids: Sequence[str]) -> None:
    if not all(ids):
        raise ValueError("request identity must be non-empty")
    if len(frozenset(ids)) < len(ids):
        raise ValueError("request identities must be unique")


# --- the live mapper's isolation contract -------------------------------------------------------


@dataclass(frozen=True)
class LiveMapperMechanism:
    """Capabilities that must all hold before mapper work overlaps target decode.

    The defaults are the one isolated configuration; ``validate`` fails closed
    on the first field (in declaration order) that departs from it.
    """

    mapper_compute_role: Literal["source", "target"] = "source"
    mapped_output_slots: int = 2
    direct_target_placement: bool = True
    target_mapper_workspace_bytes: int = 0
    target_transfer_workspace_bytes: int = 0
    scheduler_serialized_allocation: bool = True
    scheduler_serialized_publication: bool = True
    source_slot_gpu_ack: bool = True
    max_staged_transactions: int = 1

    def unmet_requirements(self) -> list[str]:
        """Messages of every isolation property this mechanism lacks."""
        out = []
        for f in fields(self):
            value, required = getattr(self, f.name), getattr(_ISOLATED, f.name)
            ok = value >= required if f.name in _AT_LEAST else value == required
            if not ok:
                out.append(_ISOLATION_MESSAGES[f.name])
        return out

    def validate(self) -> None:
        unmet = self.unmet_requirements()
        if unmet:
            raise ValueError(unmet[0])


_ISOLATED = LiveMapperMechanism()
_AT_LEAST = frozenset({"mapped_output_slots"})  # more slots than the minimum are fine
_ISOLATION_MESSAGES = {
    "mapper_compute_role": "live mapper compute must be source-isolated",
    "mapped_output_slots": "live mapper requires at least two output slots",
    "direct_target_placement": "live mapper requires direct target placement",
    "target_mapper_workspace_bytes": "live mapper cannot allocate target mapper workspace",
    "target_transfer_workspace_bytes": "live mapper cannot allocate target transfer workspace",
    "scheduler_serialized_allocation": "target allocation must be scheduler-serialized",
    "scheduler_serialized_publication": "target publication must be scheduler-serialized",
    "source_slot_gpu_ack": "source slots require target GPU-complete ACKs",
    "max_staged_transactions": "exactly one unpublished transaction is supported",
}


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


# --- routing --------------------------------------------------------------------------------------


@dataclass(frozen=True)
class _Arrival:
    requests: tuple           # after cancellations
    decoder_active: bool
    service_class: str
    cohort_preformed: bool


class OnlineMapperRouter:
    """Choose the serving path of an arrival cohort.

    The cohort is atomic: it takes one path, and a live cost policy that any
    request misses sends all of it to native re-prefill.
    """

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
        self._rules = self._build_rules()

    def _build_rules(self) -> list[tuple[str, str, Callable[[_Arrival], bool]]]:
        """(mode, reason, applies) in priority order; the last rule always applies."""
        limit, policy = self.max_cohort_requests, self.live_cost_policy
        rules = [
            ("backpressure", "cohort_canceled", lambda a: not a.requests),
            ("backpressure", "cohort_request_limit", lambda a: len(a.requests) > limit),
        ]
        if self.live_mechanism is not None:
            rules += [
                ("native_reprefill", "below_live_mapper_break_even",
                 lambda a: policy is not None and not all(map(policy.admits, a.requests))),
                ("cachebridge_live", "source_isolated_live_mapper", lambda a: True),
            ]
        return rules + [
            ("native_reprefill", "decoder_active", lambda a: a.decoder_active),
            ("native_reprefill", "latency_service_class", lambda a: a.service_class == "latency"),
            ("native_reprefill", "trickle_arrival_no_wait", lambda a: not a.cohort_preformed),
            ("cachebridge_cohort", "idle_preformed_throughput_cohort", lambda a: True),
        ]

    def route(self, requests: Iterable[MapperRequest], *, decoder_active: bool,
              service_class: Literal["latency", "throughput"], cohort_preformed: bool,
              canceled_request_ids: Iterable[str] = ()) -> RouterDecision:
        cohort = tuple(requests)
        if not cohort:
            raise ValueError("route requires at least one request")
        _require_identities([r.request_id for r in cohort])
        canceled = tuple(canceled_request_ids)
        dropped = frozenset(canceled)
        if len(dropped) < len(canceled):
            raise ValueError("canceled request identities must be unique")
        unknown = dropped.difference(r.request_id for r in cohort)
        if unknown:
            raise ValueError(f"unknown canceled request identities: {sorted(unknown)}")
        arrival = _Arrival(tuple(r for r in cohort if r.request_id not in dropped), decoder_active,
                           service_class, cohort_preformed)
        mode, reason = next((m, why) for m, why, applies in self._rules if applies(arrival))
        return RouterDecision(mode, reason, arrival.requests, canceled, decoder_active, service_class,
                              cohort_preformed)

    def dispatch(self, decision: RouterDecision, *, cachebridge_live: Callable | None = None,
                 cachebridge_cohort: Callable, native_reprefill: Callable):
        """Run exactly the one serving path the decision selected."""
        if decision.mode == "backpressure":
            raise RuntimeError(f"cannot dispatch backpressured route: {decision.reason}")
        paths = {"cachebridge_live": cachebridge_live, "cachebridge_cohort": cachebridge_cohort,
                 "native_reprefill": native_reprefill}
        path = paths[decision.mode]
        if path is None:
            raise RuntimeError(f"{decision.mode} callback is required")
        return path(decision.requests)


# --- one live (post-arrival) transaction -----------------------------------------------------------

# step -> (state it leaves from, state it enters)
_LIVE_STEPS = {
    "mark_source_complete": ("mapping", "source_ready"),
    "publish": ("source_ready", "published"),
    "mark_submitted": ("published", "idle"),
}


class LiveMapperAdmission:
    """One unpublished post-arrival mapper transaction at a time."""

    def __init__(self, *, mechanism: LiveMapperMechanism, query_reserve_tokens: int = 32) -> None:
        if query_reserve_tokens < 0:
            raise ValueError("query reserve must be non-negative")
        mechanism.validate()
        self.mechanism = mechanism
        self.query_reserve_tokens = query_reserve_tokens
        self._state = "idle"
        self._request: MapperRequest | None = None
        self._during_decode = False
        self._submitted: list[str] = []
        self._error: str | None = None

    def plan(self, request: MapperRequest, *, available_target_tokens: int,
             decoder_active: bool) -> LiveAdmissionPlan:
        _require_identities([request.request_id])
        if request.history_tokens <= 0:
            raise ValueError("history_tokens must be positive")
        need = request.history_tokens + self.query_reserve_tokens
        if self._state != "idle":
            verdict = (False, "mapper_transaction_in_flight")
        elif need > available_target_tokens:
            verdict = (False, "target_token_backpressure")
        else:
            verdict = (True, "admitted_during_decode" if decoder_active else "admitted")
        return LiveAdmissionPlan(*verdict, request, need, available_target_tokens, decoder_active)

    def begin(self, plan: LiveAdmissionPlan) -> MapperRequest:
        if self._state != "idle":
            raise RuntimeError(f"cannot begin while state={self._state}")
        if not plan.admitted:
            raise RuntimeError(f"cannot execute rejected plan: {plan.reason}")
        if plan.request.request_id in self._submitted:
            raise RuntimeError("request identity was already published")
        self._request, self._during_decode = plan.request, plan.decoder_active
        self._state, self._error = "mapping", None
        return plan.request

    def _step(self, step: str, request_id: str) -> None:
        leaves, enters = _LIVE_STEPS[step]
        owner = None if self._request is None else self._request.request_id
        if self._state != leaves or owner != request_id:
            raise RuntimeError("operation does not own the active mapper transaction")
        self._state = enters

    def mark_source_complete(self, request_id: str) -> None:
        self._step("mark_source_complete", request_id)

    def publish(self, request_id: str, proof: PublicationProof) -> None:
        leaves, _ = _LIVE_STEPS["publish"]
        if self._state == leaves and self._request is not None and self._request.request_id == request_id \
                and not (proof.gpu_reads_complete and proof.tp_vote_passed):
            self.quarantine("publication proof failed")
            raise RuntimeError("cannot publish without GPU completion and TP vote")
        self._step("publish", request_id)

    def mark_submitted(self, request_id: str) -> None:
        self._step("mark_submitted", request_id)
        self._submitted.append(request_id)
        self._clear()

    def rollback(self, request_id: str, *, gpu_reads_complete: bool, target_pages_released: bool) -> None:
        if self._request is None or self._request.request_id != request_id:
            raise RuntimeError("rollback does not own the active transaction")
        if self._state not in ("mapping", "source_ready"):
            raise RuntimeError(f"cannot roll back while state={self._state}")
        if not (gpu_reads_complete and target_pages_released):
            self.quarantine("unsafe rollback")
            raise RuntimeError("rollback requires completed reads and released pages")
        self._clear()

    def _clear(self) -> None:
        self._request, self._during_decode, self._state = None, False, "idle"

    def quarantine(self, error) -> None:
        self._state, self._error = "quarantined", str(error)

    def snapshot(self) -> dict:
        m = self.mechanism
        state = {
            "state": self._state,
            "active_request": None if self._request is None else self._request.request_id,
            "decoder_active_during_mapping": self._during_decode,
            "completed_request_ids": tuple(self._submitted),
            "error": self._error,
        }
        for name in ("mapper_compute_role", "mapped_output_slots", "max_staged_transactions",
                     "target_mapper_workspace_bytes", "target_transfer_workspace_bytes",
                     "direct_target_placement", "scheduler_serialized_publication"):
            state[name] = getattr(m, name)
        return state


# --- one admitted cohort --------------------------------------------------------------------------


class _Ledger:
    """A cohort's requests in admission order and how far publication got.

    ``requests[:cursor]`` are published; ``requests[cursor]`` is the only one
    that may be mapped next; ``active`` is its id while its transaction runs.
    """

    def __init__(self, requests: tuple = ()) -> None:
        self.requests = requests
        self.cursor = 0
        self.active: str | None = None

    @property
    def ids(self) -> tuple:
        return tuple(r.request_id for r in self.requests)

    @property
    def published(self) -> tuple:
        return self.ids[:self.cursor]

    @property
    def pending(self) -> tuple:
        return self.ids[self.cursor:]


# step -> (states it may leave from, state it enters)
_COHORT_STEPS = {
    "admit": (("idle",), "admitted"),
    "begin_next_mapper": (("admitted", "mapping"), "mapping"),
    "coalesced_query_batch": (("ready",), "dispatched"),
    "finish_queries": (("dispatched",), "idle"),
}


class OnlineMapperAdmission:
    """One admitted cohort: FIFO mapper transactions, then one query batch."""

    def __init__(self, *, max_cohort_requests: int = 4, query_reserve_tokens_per_request: int = 32) -> None:
        if max_cohort_requests <= 0:
            raise ValueError("max_cohort_requests must be positive")
        if query_reserve_tokens_per_request < 0:
            raise ValueError("query reserve must be non-negative")
        self.max_cohort_requests = max_cohort_requests
        self.query_reserve_tokens_per_request = query_reserve_tokens_per_request
        self._state = "idle"
        self._ledger = _Ledger()
        self._error: str | None = None
        self._batched_tokens = 0  # tokens of the cohort mapped in one launch, 0 for per-request maps

    def _leave(self, step: str, verb: str) -> None:
        sources, enters = _COHORT_STEPS[step]
        if self._state not in sources:
            raise RuntimeError(f"cannot {verb} while state={self._state}")
        self._state = enters

    def plan(self, requests: Iterable[MapperRequest], *, available_target_tokens: int) -> AdmissionPlan:
        cohort = tuple(requests)
        if not cohort:
            raise ValueError("cohort must be non-empty")

        def verdict(ok, reason, required):
            return AdmissionPlan(ok, reason, cohort, required, available_target_tokens, int(ok), False, True)

        if len(cohort) > self.max_cohort_requests:
            return verdict(False, "cohort_request_limit", 0)
        _require_identities([r.request_id for r in cohort])
        if min(r.history_tokens for r in cohort) <= 0:
            raise ValueError("history_tokens must be positive")
        required = sum(r.history_tokens + self.query_reserve_tokens_per_request for r in cohort)
        if required > available_target_tokens:
            return verdict(False, "target_token_backpressure", required)
        return verdict(True, "admitted", required)

    def admit(self, plan: AdmissionPlan) -> None:
        if self._state == "idle" and not plan.admitted:
            raise RuntimeError(f"cannot execute rejected plan: {plan.reason}")
        self._leave("admit", "admit")
        self._ledger, self._error, self._batched_tokens = _Ledger(plan.requests), None, 0

    def begin_next_mapper(self) -> MapperRequest:
        ledger = self._ledger
        if self._state in _COHORT_STEPS["begin_next_mapper"][0]:
            if ledger.active is not None:
                raise RuntimeError("another mapper transaction is active")
            if ledger.cursor == len(ledger.requests):
                raise RuntimeError("cohort has no pending mapper request")
        self._leave("begin_next_mapper", "start mapper")
        request = ledger.requests[ledger.cursor]
        ledger.active = request.request_id
        return request

    def publish_active_mapper(self, request_id: str) -> None:
        ledger = self._ledger
        if self._state != "mapping" or ledger.active != request_id:
            raise RuntimeError("publication does not own the active mapper transaction")
        if ledger.pending[:1] != (request_id,):
            raise RuntimeError("mapper completion violated FIFO admission order")
        ledger.cursor += 1
        ledger.active = None
        self._state = "mapping" if ledger.pending else "ready"

    def coalesced_query_batch(self) -> tuple:
        ledger = self._ledger
        if self._state != "ready" or ledger.active is not None or ledger.pending:
            raise RuntimeError("queries cannot dispatch before every prefix is published")
        if ledger.published != ledger.ids:
            raise RuntimeError("published request set differs from admitted cohort")
        self._leave("coalesced_query_batch", "dispatch queries")
        return ledger.ids

    def finish_queries(self) -> None:
        self._leave("finish_queries", "finish queries")
        self._ledger, self._batched_tokens = _Ledger(), 0

    def _run(self, plan: AdmissionPlan, *, before: Callable[[tuple], None] | None,
             each: Callable[[MapperRequest], None], query_batch: Callable[[tuple], _Result]) -> _Result:
        """Admit, optionally map the cohort, step every request FIFO, query once.

        Any failure quarantines the cohort with the failing request still
        active (or none, if ``before`` failed) and is re-raised.
        """
        self.admit(plan)
        try:
            if before is not None:
                before(self._ledger.requests)
            while self._ledger.pending:
                request = self.begin_next_mapper()
                each(request)
                self.publish_active_mapper(request.request_id)
            result = query_batch(self.coalesced_query_batch())
        except BaseException as error:
            self.quarantine(error)
            raise
        self.finish_queries()
        return result

    def execute_cohort(self, plan: AdmissionPlan, *, mapper_transaction: Callable[[MapperRequest], None],
                       query_batch: Callable[[tuple], _Result]) -> _Result:
        """One synchronous mapper transaction per request (map, install, checks
        and the TP vote inside the callback), then one query batch."""
        return self._run(plan, before=None, each=mapper_transaction, query_batch=query_batch)

    def execute_cohort_batched(self, plan: AdmissionPlan, *, map_cohort: Callable[[tuple], None],
                               publish: Callable[[MapperRequest], None],
                               query_batch: Callable[[tuple], _Result]) -> _Result:
        """Map every admitted request in one launch, then publish in FIFO order.

        ``map_cohort(requests)`` must return after the cohort's map and install
        have completed on the GPU (e.g. ``map_install_batch`` followed by a
        stream synchronization). ``publish(request)`` runs each request's safety
        checks and TP vote, in admission order. The launch's device workspace
        grows with the cohort (``BATCH_WORKSPACE_BYTES_PER_TOKEN`` per token);
        ``snapshot`` reports it while the cohort is held.
        """
        def before(requests):
            self._batched_tokens = sum(r.history_tokens for r in requests)
            map_cohort(requests)

        return self._run(plan, before=before, each=publish, query_batch=query_batch)

    def quarantine(self, error) -> None:
        self._state, self._error = "quarantined", str(error)

    def snapshot(self) -> dict:
        ledger = self._ledger
        return {
            "state": self._state,
            "active_request": ledger.active,
            "pending_request_ids": ledger.pending,
            "published_request_ids": ledger.published,
            "error": self._error,
            "max_mapper_transactions_in_flight": 1,
            "mapper_workspace_scales_with_cohort": self._batched_tokens > 0,
            "mapper_workspace_bytes": BATCH_WORKSPACE_BYTES_PER_TOKEN * self._batched_tokens,
            "query_coalescing": True,
        }
