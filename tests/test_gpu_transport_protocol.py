"""GPU parity of the Transport mailbox protocol against its CPU oracle.

The device runs the reference's own protocol test sequences (probe kernel), the drain and
rejection cases, and full ffn_shim transactions around the Dense step; every observation is
compared with oracle/transport_protocol.py on the same sequence and with the reference
tests' literal expectations (tests/suites/cext/transport/view_test.cu:154-248,
instance_test.cu:84-115, shutdown_test.cu:195-252).  Every kernel here exits by itself:
the one wait (completion) is bounded, and the timeout case is forced from the host by
never launching the agent side, with a 100 us deadline.
"""

from __future__ import annotations

import pytest
import torch

from crosspool_amd.agent import FfnAgent
from crosspool_amd.ffn import DpRowLayout, ForwardMode, OutputRequirement, ResultCode
from crosspool_amd.ops import attach, attached_transport, detach, ffn_shim
from crosspool_amd.transport import FfnRequestMetadata, MailboxStatus, TransportResident
from crosspool_amd.weights import DenseFfnWeights
from oracle import ffn_oracle as o
from oracle import transport_protocol as tp
from parity import assert_bitwise_equal, assert_ffn_parity, slots_tensor, to_device

from test_transport_oracle import VIEW_TEST_EXPECTED

pytestmark = pytest.mark.gpu

DECODE = FfnRequestMetadata(0, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE, DpRowLayout.NONE)
WORDS = {0: 11, 1: 1, 2: 3, 3: 4, 4: 4, 5: 2, 6: 3}


def _is_nan(tensor: torch.Tensor) -> bool:
    return bool(torch.isnan(tensor.float()).all())


@pytest.mark.parametrize("number", sorted(VIEW_TEST_EXPECTED))
def test_probe_matches_view_test(device, number):
    print(f"probe scenario {number}", flush=True)
    with TransportResident(device, [(4, 1)]) as transport:
        observed = transport.probe(0, number)[: WORDS[number]]
        assert observed == tp.scenario(number, tp.Arena(payload_row_capacity=4))
        assert observed == [int(v) for v in VIEW_TEST_EXPECTED[number]]
        assert transport.snapshot(0).violations == 0


def test_open_and_drain_every_arena(device):
    # shutdown_test.cu:195-219
    with TransportResident(device, [(1, 1), (1, 1)]) as transport:
        assert transport.snapshot(0).mailbox_status is MailboxStatus.DORMANT
        transport.open()
        assert [transport.snapshot(i).mailbox_status for i in (0, 1)] == [MailboxStatus.IDLE] * 2
        transport.drain()
        for index in (0, 1):
            state = transport.snapshot(index)
            assert state.shutdown and state.mailbox_status is MailboxStatus.CLOSED
            assert state.generation_failure is ResultCode.OK and state.violations == 0


def test_published_rejection_drains_idle_peer(device):
    # shutdown_test.cu:221-252, with the agent side answering through evaluate.
    with TransportResident(device, [(1, 1), (1, 1)]) as transport:
        transport.open()
        arenas = [tp.Arena(payload_row_capacity=1) for _ in range(2)]
        for arena in arenas:
            arena.open()
        assert transport.probe(0, 5)[:2] == tp.scenario(5, arenas[0])
        transport.evaluate(0)
        tp.evaluate(arenas, 0)
        first, second = transport.snapshot(0), transport.snapshot(1)
        assert first.mailbox_status is MailboxStatus.EVALUATED
        assert first.result_code == ResultCode.PROTOCOL_MISMATCH
        assert second.mailbox_status is MailboxStatus.CLOSED and second.shutdown
        assert transport.probe(0, 6)[:3] == tp.scenario(6, arenas[0])
        assert transport.snapshot(0).mailbox_status is MailboxStatus.CLOSED
        assert transport.snapshot(0).violations == 0 and transport.snapshot(1).violations == 0


def test_rejects_before_staging_after_canonical_failure(device):
    # instance_test.cu:97-115: NaN output, mailbox still Dormant, failure kept.
    with TransportResident(device, [(2, 1)]) as transport:
        transport.publish_failure(0, ResultCode.PROTOCOL_MISMATCH)
        output = torch.ones((2, 2), dtype=torch.bfloat16, device=device)
        transport.submit(0, 2, DECODE)
        transport.complete(0, output)
        state = transport.snapshot(0)
        assert _is_nan(output)
        assert state.mailbox_status is MailboxStatus.DORMANT
        assert state.generation_failure is ResultCode.PROTOCOL_MISMATCH
        assert state.instance_outcome is ResultCode.PROTOCOL_MISMATCH and state.violations == 0


def test_rejects_before_staging_after_shutdown(device):
    # instance_test.cu:84-95 (shutdown published by a drain here).
    with TransportResident(device, [(2, 1)]) as transport:
        transport.open()
        transport.drain()
        output = torch.ones((2, 2), dtype=torch.bfloat16, device=device)
        transport.submit(0, 2, DECODE)
        transport.complete(0, output)
        state = transport.snapshot(0)
        assert _is_nan(output) and state.instance_outcome is ResultCode.SHUTDOWN
        assert state.mailbox_status is MailboxStatus.CLOSED and state.violations == 0


def test_transaction_lifecycle_and_dp_rows(device):
    with TransportResident(device, [(16, 2)]) as transport:
        transport.open()
        arena = tp.Arena(payload_row_capacity=16, atn_dp_size=2)
        arena.open()
        metadata = FfnRequestMetadata(7, ForwardMode.PREFILL, OutputRequirement.PER_RANK_COMPLETE,
                                      DpRowLayout.PACKED_BY_RANK)
        rows = torch.tensor([5, 11], dtype=torch.int64, device=device)
        output = torch.zeros((16, 8), dtype=torch.bfloat16, device=device)
        transport.submit(0, 16, metadata, rows)
        published = transport.snapshot(0)
        assert tp.submit(arena, 16, tp.Request(7, 1, 1, 2), [5, 11]) == tp.PENDING
        assert published.mailbox_status is MailboxStatus.PUBLISHED and published.instance_outcome is None
        assert published.payload_rows == 16 and published.request == (7, 1, 1, 2)
        assert published.dp_rank_payload_rows == (5, 11)
        transport.evaluate(0)
        assert tp.evaluate([arena], 0) == ResultCode.OK
        assert transport.snapshot(0).mailbox_status is MailboxStatus.EVALUATED
        transport.complete(0, output)
        assert tp.complete(arena) == (ResultCode.OK, False)
        done = transport.snapshot(0)
        assert done.mailbox_status is MailboxStatus.IDLE and done.instance_outcome is ResultCode.OK
        assert done.payload_rows == 0 and done.request == (0, 0, 0, 0)
        assert done.result_code == ResultCode.PROTOCOL_MISMATCH and done.violations == 0
        assert not torch.isnan(output.float()).any()


def test_completion_times_out_without_agent(device):
    # The agent side never runs: the bounded wait ends, Timeout becomes the canonical
    # failure (the reference traps here) and the output is NaN-filled.
    with TransportResident(device, [(4, 1)]) as transport:
        transport.open()
        output = torch.zeros((4, 8), dtype=torch.bfloat16, device=device)
        transport.submit(0, 4, DECODE)
        transport.complete(0, output, timeout_ns=100_000)
        state = transport.snapshot(0)
        assert _is_nan(output)
        assert state.generation_failure is ResultCode.TIMEOUT and state.instance_outcome is ResultCode.TIMEOUT
        assert state.mailbox_status is MailboxStatus.PUBLISHED and state.violations == 0


def test_repeated_open_counts_a_violation(device):
    # The reference traps on a second open (protocol.cuh:22-25); the device counts it and
    # publishes the canonical ProtocolMismatch.
    with TransportResident(device, [(4, 1)]) as transport:
        transport.open()
        transport.open()
        state = transport.snapshot(0)
        assert state.violations == 1 and state.generation_failure is ResultCode.PROTOCOL_MISMATCH
        with pytest.raises(tp.ReferenceAbort):
            arena = tp.Arena(payload_row_capacity=4)
            arena.open()
            arena.open()


def _agent(device, hidden, intermediate, seed, capacity):
    w_gate_up, w_down, _ = o.generate_layer(hidden, intermediate, seed)
    agent = FfnAgent(device)
    agent.register_layer(
        instance_index=0, layer_ordinal=0,
        weights=DenseFfnWeights.from_tensors(to_device(w_gate_up, device), to_device(w_down, device)),
    )
    agent.materialize(maximum_row_capacity=capacity)
    return agent, w_gate_up, w_down


def test_shim_mailbox_matches_direct_path(device):
    # Many transactions queued without a host sync: every output equals the direct path's
    # bits, meets the FFN parity bar, and the mailbox ends Idle with no violation.
    hidden, intermediate = 1024, 3072
    agent, w_gate_up, w_down = _agent(device, hidden, intermediate, 18, 64)
    try:
        inputs = [o.generate_hidden_states(rows, hidden, 80 + rows) for rows in (1, 5, 64, 17, 1, 33)]
        outputs = {}
        for mode in ("settle", "lane_stream", "direct"):
            attach(agent, mailbox=mode != "direct", lane_stream=mode == "lane_stream")
            outputs[mode] = [ffn_shim(to_device(x, device), None, DECODE) for x in inputs]
            torch.cuda.synchronize()
            if mode != "direct":
                state = attached_transport().snapshot(0)
                assert state.mailbox_status is MailboxStatus.IDLE and state.violations == 0
                assert state.instance_outcome is ResultCode.OK
            detach()
        for index, x in enumerate(inputs):
            direct = outputs["direct"][index].cpu()
            for mode in ("settle", "lane_stream"):
                assert_bitwise_equal(outputs[mode][index].cpu(), direct)
            assert_ffn_parity(direct, o.dense_partial_reference(x, w_gate_up, w_down), o.dense_fp32(x, w_gate_up, w_down))
    finally:
        detach()
        agent.close()


def test_shim_lane_fault_is_a_canonical_failure(device):
    # A Lane fault (a slot outside the mailbox in an earlier replay) makes the agent answer
    # ProtocolMismatch: NaN output, the arena drained, later requests rejected as Shutdown.
    hidden, intermediate = 256, 512
    agent, _, _ = _agent(device, hidden, intermediate, 21, 8)
    try:
        pool = to_device(o.generate_hidden_states(4, hidden, 3), device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool, slots=slots_tensor([0, 9], device))
        agent.lanes[0].synchronize()
        x = to_device(o.generate_hidden_states(3, hidden, 4), device)
        for lane_stream in (False, True):
            attach(agent, lane_stream=lane_stream)
            first = ffn_shim(x, None, DECODE)
            second = ffn_shim(x, None, DECODE)
            torch.cuda.synchronize()
            assert _is_nan(first) and _is_nan(second)
            state = attached_transport().snapshot(0)
            assert state.shutdown and state.mailbox_status is MailboxStatus.CLOSED
            assert state.instance_outcome is ResultCode.SHUTDOWN and state.violations == 0
            detach()
        arenas = [tp.Arena(payload_row_capacity=8)]
        arenas[0].open()
        assert tp.instance_transaction(arenas, 0, 3, tp.DECODE_REQUEST, lane_fault=True) == (
            ResultCode.PROTOCOL_MISMATCH, True)
        assert tp.instance_transaction(arenas, 0, 3, tp.DECODE_REQUEST) == (ResultCode.SHUTDOWN, True)
    finally:
        detach()
        agent.close()
