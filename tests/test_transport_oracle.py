"""CPU pins of the Transport mailbox oracle (oracle/transport_protocol.py).

The expected values are the reference's own device-test assertions, restated as known
answers (paths relative to the CrossPool checkout):

* tests/suites/cext/transport/view_test.cu:154-248 (five lifecycle scenarios);
* tests/suites/cext/transport/protocol_test.cpp:20-34 (request metadata validity);
* tests/suites/cext/transport/instance_test.cu:84-115 (rejection before staging);
* tests/suites/cext/transport/shutdown_test.cu:195-252 (drain of every arena).

Mutated copies of the oracle (a transition that forgets to reset, a wrong precedence)
must fail these pins, which shows they discriminate.
"""

from __future__ import annotations

import pytest

from oracle import transport_protocol as tp
from oracle.transport_protocol import MailboxStatus as S
from oracle.transport_protocol import Result as R

# view_test.cu:167-177, 189-190, 206-208, 224-226, 241-243
VIEW_TEST_EXPECTED = {
    0: [S.DORMANT, S.IDLE, 1, S.PUBLISHED, S.EVALUATED, R.OK, S.IDLE, R.PROTOCOL_MISMATCH, 0, 1, S.CLOSED],
    1: [R.TIMEOUT],
    2: [1, S.CLOSED, R.SHUTDOWN],
    3: [1, S.CLOSED, R.PROTOCOL_MISMATCH, R.PROTOCOL_MISMATCH],
    4: [1, S.CLOSED, R.OK, 1],
}


@pytest.mark.parametrize("number", sorted(VIEW_TEST_EXPECTED))
def test_view_test_scenarios(number):
    arena = tp.Arena(payload_row_capacity=4)
    assert tp.scenario(number, arena) == VIEW_TEST_EXPECTED[number]


def test_request_metadata_validity():
    # protocol_test.cpp:20-34
    valid = tp.Request(0, 2, 1, 0)
    assert valid.valid()
    assert not tp.Request(0, 99, 1, 0).valid()
    assert not tp.Request(0, 2, 99, 0).valid()
    assert not tp.Request(0, 2, 1, 99).valid()
    assert not tp.Request().valid()  # a zero-initialised request is not publishable


def _opened(*capacities, dp=1):
    arenas = [tp.Arena(payload_row_capacity=c, atn_dp_size=dp) for c in capacities]
    for arena in arenas:
        arena.open()
    return arenas


def test_rejects_before_staging_after_shutdown():
    # instance_test.cu:84-95: the shutdown flag alone rejects the request; output is NaN.
    arena = tp.Arena(payload_row_capacity=2)
    arena.publish_shutdown()
    assert tp.submit(arena, 2, tp.DECODE_REQUEST) == R.SHUTDOWN
    assert tp.complete(arena) == (R.SHUTDOWN, True)


def test_rejects_before_staging_after_canonical_failure():
    # instance_test.cu:97-115: NaN output, the mailbox stays Dormant, the failure stays.
    arena = tp.Arena(payload_row_capacity=2)
    arena.publish_generation_failure(R.PROTOCOL_MISMATCH)
    tp.submit(arena, 2, tp.DECODE_REQUEST)
    assert tp.complete(arena) == (R.PROTOCOL_MISMATCH, True)
    assert arena.status == S.DORMANT
    assert arena.generation_failure == R.PROTOCOL_MISMATCH


def test_drain_closes_every_arena():
    # shutdown_test.cu:195-219
    arenas = _opened(1, 1)
    tp.drain(arenas)
    assert [a.shutdown for a in arenas] == [True, True]
    assert [a.status for a in arenas] == [S.CLOSED, S.CLOSED]
    assert [a.generation_failure for a in arenas] == [R.OK, R.OK]


def test_published_rejection_drains_idle_peer():
    # shutdown_test.cu:221-252: an over-capacity request is answered with ProtocolMismatch,
    # the drain closes the idle peer, the producer then closes its own evaluated request.
    arenas = _opened(1, 1)
    assert tp.scenario(5, arenas[0]) == [1, S.PUBLISHED]
    assert tp.evaluate(arenas, 0) == R.PROTOCOL_MISMATCH
    assert arenas[1].status == S.CLOSED
    assert tp.scenario(6, arenas[0]) == [S.EVALUATED, R.PROTOCOL_MISMATCH, S.CLOSED]
    assert [a.status for a in arenas] == [S.CLOSED, S.CLOSED]


def test_transactions_acknowledge_and_reset():
    arenas = _opened(8)
    for rows in (1, 8, 3):
        assert tp.instance_transaction(arenas, 0, rows, tp.Request(5, 1, 1, 0)) == (R.OK, False)
        assert arenas[0].status == S.IDLE
        assert arenas[0].payload_rows == 0 and arenas[0].request == tp.Request()
        assert arenas[0].result_code == R.PROTOCOL_MISMATCH


def test_invalid_request_and_lane_fault_are_mismatches():
    arenas = _opened(8, 8)
    # A published request over capacity cannot come through submit's host checks, but the
    # agent side still validates what it reads.
    assert tp.instance_transaction(arenas, 0, 9, tp.DECODE_REQUEST) == (R.PROTOCOL_MISMATCH, True)
    assert arenas[0].status == S.CLOSED and arenas[1].status == S.CLOSED
    assert all(a.shutdown for a in arenas)
    assert tp.instance_transaction(arenas, 1, 1, tp.DECODE_REQUEST) == (R.SHUTDOWN, True)
    arenas = _opened(8)
    assert tp.instance_transaction(arenas, 0, 2, tp.DECODE_REQUEST, lane_fault=True) == (R.PROTOCOL_MISMATCH, True)


def test_dp_layout_rules():
    arenas = _opened(8, dp=2)
    assert tp.instance_transaction(arenas, 0, 4, tp.Request(0, 2, 1, 2), [1, 3]) == (R.OK, False)
    assert arenas[0].dp_rank_payload_rows == [1, 3]
    assert tp.instance_transaction(arenas, 0, 4, tp.Request(0, 2, 1, 0), [1, 3]) == (R.PROTOCOL_MISMATCH, True)


def test_successful_result_survives_shutdown():
    arenas = _opened(4)
    tp.submit(arenas[0], 2, tp.DECODE_REQUEST)
    tp.evaluate(arenas, 0)
    arenas[0].publish_shutdown()
    assert tp.complete(arenas[0]) == (R.OK, False)
    assert arenas[0].status == S.CLOSED


def test_reference_aborts():
    arena = tp.Arena(payload_row_capacity=4)
    with pytest.raises(tp.ReferenceAbort):
        tp.submit(arena, 1, tp.DECODE_REQUEST)  # a Dormant mailbox refuses the claim
    arena = tp.Arena(payload_row_capacity=4)
    arena.open()
    with pytest.raises(tp.ReferenceAbort):
        arena.open()
    with pytest.raises(tp.ReferenceAbort):
        arena.publish_result(R.OK)
    with pytest.raises(tp.ReferenceAbort):
        arena.publish_generation_failure(R.SHUTDOWN)
    arena.publish_generation_failure(R.TIMEOUT)
    with pytest.raises(tp.ReferenceAbort):
        arena.publish_generation_failure(R.PROTOCOL_MISMATCH)
    arena = tp.Arena(payload_row_capacity=4)
    arena.open()
    tp.submit(arena, 1, tp.DECODE_REQUEST)
    with pytest.raises(tp.ReferenceAbort):
        tp.complete(arena, published_answered=False)  # a silent agent without a canonical failure


def test_pins_reject_planted_mistakes(monkeypatch):
    # Acknowledge that forgets to reset the request facts.
    def sloppy_acknowledge(self):
        self.status = S.IDLE

    monkeypatch.setattr(tp.Arena, "acknowledge", sloppy_acknowledge)
    assert tp.scenario(0, tp.Arena(payload_row_capacity=4)) != VIEW_TEST_EXPECTED[0]
    monkeypatch.undo()

    # Precedence: an Ok mailbox result wins over a canonical failure published after it
    # (instance.cu:155-159); a completion that let the failure win would return TIMEOUT.
    arenas = _opened(4)
    tp.submit(arenas[0], 1, tp.DECODE_REQUEST)
    tp.evaluate(arenas, 0)
    arenas[0].publish_generation_failure(R.TIMEOUT)
    assert tp.complete(arenas[0]) == (R.OK, False)

    # A drain that forgets the idle peer.
    monkeypatch.setattr(tp, "finish_terminal_mailbox", lambda arena: None)
    arenas = _opened(1, 1)
    tp.drain(arenas)
    assert [a.status for a in arenas] != [S.CLOSED, S.CLOSED]
