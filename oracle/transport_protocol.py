"""CPU restatement of the Transport mailbox protocol.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Pure-Python state machine of
one rank-local request mailbox and its arena words, restating (paths relative to the
CrossPool checkout):

* the lifecycle and transitions, src/cext-include/xpool/transport/protocol.hpp:33-87 and
  protocol.cuh:14-68;
* the sticky arena words, src/cext-include/xpool/transport/arena.hpp (ArenaState) and
  arena.cuh:50-63;
* the Instance transaction, src/cext/transport/instance.cu:36-201;
* the Resident's request validation, service and drain, src/cext/transport/atnagent.cu:20-186.

Where the reference calls ``xpool::abort_if`` this restatement raises
:class:`ReferenceAbort`; the device build instead counts a violation and publishes the
canonical ProtocolMismatch failure, and the tests check that it does so exactly where
this module raises.

Pinned by the reference's own device tests, restated as known answers in
tests/test_transport_oracle.py: the five scenarios of
tests/suites/cext/transport/view_test.cu:154-248, the two of instance_test.cu:84-115 and
the two drain cases of shutdown_test.cu:195-252, plus RequestMetadata validity
(protocol_test.cpp:20-34).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import IntEnum

__all__ = [
    "MailboxStatus",
    "Result",
    "ReferenceAbort",
    "Request",
    "Arena",
    "request_valid",
    "submit",
    "evaluate",
    "complete",
    "drain",
    "instance_transaction",
    "scenario",
]


class MailboxStatus(IntEnum):
    """protocol.hpp:33-49."""

    DORMANT = 0
    IDLE = 1
    STAGING = 2
    PUBLISHED = 3
    EVALUATED = 4
    CLOSED = 5


class Result(IntEnum):
    """ffn.hpp:43-48."""

    OK = 0
    SHUTDOWN = 1
    PROTOCOL_MISMATCH = 2
    TIMEOUT = 3


PENDING = 0xFFFFFFFF


class ReferenceAbort(AssertionError):
    """A precondition the reference guards with ``xpool::abort_if`` does not hold."""


def _require(condition: bool, what: str) -> None:
    if not condition:
        raise ReferenceAbort(what)


@dataclass(frozen=True)
class Request:
    """RequestMetadata (protocol.hpp:14-29); zero-initialised fields are invalid."""

    layer_ordinal: int = 0
    forward_mode: int = 0
    output_requirement: int = 0
    dp_row_layout: int = 0

    def valid(self) -> bool:
        """protocol.hpp:25-28 over ffn.hpp:56-70."""

        return (
            self.forward_mode in (1, 2, 4)
            and self.output_requirement in (1, 2)
            and self.dp_row_layout in (0, 1, 2)
        )


DECODE_REQUEST = Request(0, 2, 1, 0)


@dataclass
class Arena:
    """One arena: mailbox (protocol.hpp:52-62), ArenaState and the staged DP rows."""

    payload_row_capacity: int
    atn_dp_size: int = 1
    status: int = MailboxStatus.DORMANT
    result_code: int = Result.OK
    payload_rows: int = 0
    request: Request = field(default_factory=Request)
    shutdown: bool = False
    generation_failure: int = Result.OK
    dp_rank_payload_rows: list[int] = field(default_factory=list)
    instance_outcome: int = Result.OK

    # ---- arena.cuh:50-63
    def publish_generation_failure(self, code: int) -> None:
        _require(code in (Result.PROTOCOL_MISMATCH, Result.TIMEOUT), "only mismatch or timeout are canonical")
        observed = self.generation_failure
        if observed == Result.OK:
            self.generation_failure = code
        _require(observed in (Result.OK, code), "a different canonical failure is already published")

    def publish_shutdown(self) -> None:
        self.shutdown = True

    # ---- protocol.cuh:14-68
    def observe(self) -> int:
        _require(MailboxStatus.DORMANT <= self.status <= MailboxStatus.CLOSED, "status outside the lifecycle")
        return self.status

    def open(self) -> None:
        _require(self.observe() == MailboxStatus.DORMANT, "open needs Dormant")
        self.status = MailboxStatus.IDLE

    def try_begin_staging(self) -> bool:
        observed = self.status
        if observed == MailboxStatus.IDLE:
            self.status = MailboxStatus.STAGING
        _require(MailboxStatus.DORMANT <= observed <= MailboxStatus.CLOSED, "status outside the lifecycle")
        return observed == MailboxStatus.IDLE

    def publish_request(self) -> None:
        _require(
            self.observe() == MailboxStatus.STAGING and self.payload_rows != 0 and self.request.valid(),
            "publish needs Staging, rows and valid metadata",
        )
        self.status = MailboxStatus.PUBLISHED

    def publish_result(self, code: int) -> None:
        _require(self.observe() == MailboxStatus.PUBLISHED, "a result needs Published")
        self.result_code = code
        self.status = MailboxStatus.EVALUATED

    def acknowledge(self) -> None:
        _require(self.observe() == MailboxStatus.EVALUATED, "acknowledge needs Evaluated")
        self.result_code = Result.PROTOCOL_MISMATCH
        self.payload_rows = 0
        self.request = Request()
        self.status = MailboxStatus.IDLE

    def close_staging(self) -> None:
        _require(self.observe() == MailboxStatus.STAGING, "close_staging needs Staging")
        self.status = MailboxStatus.CLOSED

    def close_evaluated(self) -> None:
        _require(self.observe() == MailboxStatus.EVALUATED, "close_evaluated needs Evaluated")
        self.status = MailboxStatus.CLOSED

    def try_close_idle(self) -> bool:
        observed = self.status
        if observed == MailboxStatus.IDLE:
            self.status = MailboxStatus.CLOSED
        _require(MailboxStatus.DORMANT <= observed <= MailboxStatus.CLOSED, "status outside the lifecycle")
        return observed == MailboxStatus.IDLE


def request_valid(arena: Arena) -> bool:
    """atnagent.cu:34-46: an arena carries DP rows exactly when atn_dp_size > 1."""

    layout_ok = (
        arena.request.dp_row_layout == 0 if arena.atn_dp_size == 1 else arena.request.dp_row_layout in (1, 2)
    )
    return arena.request.valid() and 0 < arena.payload_rows <= arena.payload_row_capacity and layout_ok


def submit(arena: Arena, payload_rows: int, request: Request, dp_rows: list[int] | None = None) -> int:
    """Claim, stage and publish (instance.cu:46-128); returns PENDING or the terminal result."""

    failure = arena.generation_failure
    if failure != Result.OK or arena.shutdown:
        arena.instance_outcome = failure if failure != Result.OK else Result.SHUTDOWN
        return arena.instance_outcome
    if not arena.try_begin_staging():
        _require(arena.observe() == MailboxStatus.CLOSED, "only a terminal arena refuses the claim")
        failure = arena.generation_failure
        _require(failure != Result.OK or arena.shutdown, "a closed arena carries a failure or shutdown")
        arena.instance_outcome = failure if failure != Result.OK else Result.SHUTDOWN
        return arena.instance_outcome
    if dp_rows:
        for value in dp_rows:
            _require(0 <= value <= 0xFFFFFFFF, "DP row counts fit uint32")
        arena.dp_rank_payload_rows = list(dp_rows)
    arena.payload_rows = payload_rows
    arena.request = request
    failure = arena.generation_failure
    if failure != Result.OK or arena.shutdown:
        outcome = failure if failure != Result.OK else Result.SHUTDOWN
        arena.result_code = outcome
        arena.close_staging()
        arena.instance_outcome = outcome
        return outcome
    arena.publish_request()
    arena.instance_outcome = PENDING
    return PENDING


def finish_terminal_mailbox(arena: Arena) -> None:
    """atnagent.cu:92-120."""

    status = arena.observe()
    if status == MailboxStatus.IDLE:
        arena.try_close_idle()
    elif status == MailboxStatus.PUBLISHED:
        failure = arena.generation_failure
        arena.publish_result(failure if failure != Result.OK else Result.SHUTDOWN)
    else:
        _require(status != MailboxStatus.DORMANT, "drain of a mailbox that never opened")


def drain(arenas: list[Arena]) -> None:
    """Resident drain (atnagent.cu:136-147): shutdown, then each mailbox."""

    for arena in arenas:
        arena.publish_shutdown()
        finish_terminal_mailbox(arena)


def evaluate(arenas: list[Arena], index: int, lane_fault: bool = False) -> int | None:
    """Agent side of one request (atnagent.cu:48-90, 155-170); None when nothing was published."""

    arena = arenas[index]
    status = arena.observe()
    if status != MailboxStatus.PUBLISHED:
        _require(status != MailboxStatus.DORMANT, "evaluate of a mailbox that never opened")
        return None
    result = Result.OK if request_valid(arena) and not lane_fault else Result.PROTOCOL_MISMATCH
    arena.publish_result(result)
    if result != Result.OK:
        drain(arenas)
    return result


def complete(arena: Arena, *, published_answered: bool = True) -> tuple[int, bool]:
    """Result observation and acknowledgement (instance.cu:130-201).

    Returns (result, output_is_canonical_failure).  ``published_answered`` False models a
    wait that times out: the reference traps unless a canonical failure explains it.
    """

    outcome = arena.instance_outcome
    if outcome != PENDING:
        return outcome, True
    status = arena.observe()
    if status not in (MailboxStatus.EVALUATED, MailboxStatus.CLOSED) or not published_answered:
        failure = arena.generation_failure
        _require(failure != Result.OK, "timed out without a canonical failure")
        arena.instance_outcome = failure
        return failure, True
    _require(status == MailboxStatus.EVALUATED, "only the Instance closes its published request")
    failure = arena.generation_failure
    mailbox_result = arena.result_code
    result = mailbox_result if mailbox_result == Result.OK or failure == Result.OK else failure
    arena.instance_outcome = result
    if result != Result.OK:
        arena.close_evaluated()
        return result, True
    if arena.shutdown:
        arena.close_evaluated()
    else:
        arena.acknowledge()
    return result, False


def instance_transaction(
    arenas: list[Arena], index: int, payload_rows: int, request: Request, dp_rows: list[int] | None = None,
    *, lane_fault: bool = False,
) -> tuple[int, bool]:
    """submit -> evaluate -> complete, the order the single-GPU build runs them in."""

    submit(arenas[index], payload_rows, request, dp_rows)
    evaluate(arenas, index, lane_fault)
    return complete(arenas[index])


def scenario(number: int, arena: Arena) -> list[int]:
    """The reference's device-side protocol test sequences, as the probe kernel runs them.

    0-4: view_test.cu:68-150; 5, 6: shutdown_test.cu:173-191.  Returns the observation
    words in the probe's order.
    """

    if number == 0:
        observed = [arena.observe()]
        arena.open()
        observed.append(arena.observe())
        observed.append(int(arena.try_begin_staging()))
        arena.payload_rows = 2
        arena.request = Request(3, 2, 1, 0)
        arena.publish_request()
        observed.append(arena.observe())
        arena.publish_result(Result.OK)
        observed += [arena.observe(), arena.result_code]
        arena.acknowledge()
        observed += [arena.observe(), arena.result_code, arena.payload_rows]
        observed.append(int(arena.try_close_idle()))
        observed.append(arena.observe())
        return observed
    if number == 1:
        arena.publish_generation_failure(Result.TIMEOUT)
        arena.publish_generation_failure(Result.TIMEOUT)
        return [arena.generation_failure]
    if number == 2:
        arena.open()
        observed = [int(arena.try_begin_staging())]
        arena.result_code = Result.SHUTDOWN
        arena.close_staging()
        return observed + [arena.observe(), arena.result_code]
    if number in (3, 4):
        arena.open()
        observed = [int(arena.try_begin_staging())]
        arena.payload_rows = 1
        arena.request = DECODE_REQUEST
        arena.publish_request()
        if number == 3:
            arena.publish_generation_failure(Result.PROTOCOL_MISMATCH)
            arena.publish_result(Result.PROTOCOL_MISMATCH)
            arena.close_evaluated()
            return observed + [arena.observe(), arena.result_code, arena.generation_failure]
        arena.publish_result(Result.OK)
        arena.publish_shutdown()
        arena.close_evaluated()
        return observed + [arena.observe(), arena.result_code, int(arena.shutdown)]
    if number == 5:
        acquired = arena.try_begin_staging()
        _require(acquired, "the producer claims an Idle mailbox")
        arena.payload_rows = arena.payload_row_capacity + 1
        arena.request = DECODE_REQUEST
        arena.publish_request()
        return [1, arena.observe()]
    if number == 6:
        observed = [arena.observe(), arena.result_code]
        _require(
            observed[0] == MailboxStatus.EVALUATED and observed[1] == Result.PROTOCOL_MISMATCH,
            "the consumer expects a rejected request",
        )
        arena.close_evaluated()
        return observed + [arena.observe()]
    raise ValueError(f"unknown scenario {number}")
