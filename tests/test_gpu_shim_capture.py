"""``ffn_shim`` recorded inside a caller's ``torch.cuda.graph``.

The reference promises that the shim "remains safe to capture in an outer CUDA Graph"
(src/xpool/ops.py:38-39): SGLang records its decode step as a graph, shim call included.
Each mode of the shim is captured once and replayed with new inputs written into the
captured input tensor, with eager calls and host synchronisations between the replays:

* direct: the Dense step on the caller's stream;
* mailbox: the Transport transaction and the Dense step on the caller's stream;
* mailbox on the Lane stream: the step and the answer on the Lane's stream, joined back to
  the caller's stream by events (the Lane stream joins the capture);

each with the Lane's replays as direct kernel launches and as hipGraph dispatch (under a
capture the Lane launches its template's kernels directly, so they become nodes of the
caller's graph).  Every replay must equal an eager call on the same input bit for bit, the
mailbox must be Idle with an OK outcome and no violation after each replay, capture must
allocate only the output tensor (from the caller's graph pool) and take no more device memory
outside that pool than the HIP runtime takes to capture and instantiate a graph of plain
torch kernels, and replays must allocate nothing at all.
"""

from __future__ import annotations

import pytest
import torch

from crosspool_amd.agent import FfnAgent
from crosspool_amd.ffn import DpRowLayout, ForwardMode, OutputRequirement, ResultCode
from crosspool_amd.ops import attach, attached_transport, detach, ffn_shim
from crosspool_amd.transport import FfnRequestMetadata, MailboxStatus
from crosspool_amd.weights import DenseFfnWeights
from oracle import ffn_oracle as o
from parity import assert_bitwise_equal, assert_ffn_parity, to_device

pytestmark = pytest.mark.gpu

DECODE = FfnRequestMetadata(0, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE, DpRowLayout.NONE)
# Allocation granularity of the device memory the HIP runtime takes for a graph.
RUNTIME_SLACK_BYTES = 2 << 20


def _capture(device, record):
    """Capture ``record()``; the graph, its result, the device memory the capture took outside
    torch's caching allocator and the number of tensors torch allocated meanwhile."""

    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info(device)[0]
    reserved_before = torch.cuda.memory_reserved(device)
    allocations = torch.cuda.memory_stats(device)["allocation.all.allocated"]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        result = record()
    torch.cuda.synchronize()
    taken = free_before - torch.cuda.mem_get_info(device)[0]
    outside = taken - (torch.cuda.memory_reserved(device) - reserved_before)
    return graph, result, outside, torch.cuda.memory_stats(device)["allocation.all.allocated"] - allocations


def _clean(transport) -> None:
    if transport is None:
        return
    state = transport.snapshot(0)
    assert state.mailbox_status is MailboxStatus.IDLE
    assert state.instance_outcome is ResultCode.OK
    assert state.violations == 0 and not state.shutdown


@pytest.mark.parametrize("graph_dispatch", (False, True), ids=("direct_launch", "graph_dispatch"))
@pytest.mark.parametrize("mode", ("direct", "mailbox", "lane_stream"))
@pytest.mark.parametrize("rows", (3, 40))
def test_ffn_shim_replays_inside_a_captured_graph(device, mode, graph_dispatch, rows):
    print(f"shim capture mode={mode} graph_dispatch={graph_dispatch} rows={rows}", flush=True)
    hidden, intermediate = 1024, 3072
    w_gate_up, w_down, _ = o.generate_layer(hidden, intermediate, 18)
    agent = FfnAgent(device, graph_dispatch=graph_dispatch)
    try:
        agent.register_layer(
            instance_index=0, layer_ordinal=0,
            weights=DenseFfnWeights.from_tensors(to_device(w_gate_up, device), to_device(w_down, device)),
        )
        agent.materialize(maximum_row_capacity=64)
        attach(agent, mailbox=mode != "direct", lane_stream=mode == "lane_stream")
        transport = attached_transport()
        inputs = [o.generate_hidden_states(rows, hidden, 300 + index) for index in range(4)]
        static_x = to_device(inputs[0], device)

        # Warm up on a side stream, as torch.cuda.graph expects.
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            for _ in range(2):
                ffn_shim(static_x, None, DECODE)
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize()
        _clean(transport)

        # What the runtime takes for a graph of as many plain kernels as the shim records.
        scratch = torch.zeros(1024, device=device)

        def plain_kernels():
            for _ in range(8):
                scratch.add_(1.0)
            return None

        # (torch's capture itself allocates its RNG state tensors: counted by the plain graph)
        _, _, runtime_bytes, capture_allocations = _capture(device, plain_kernels)
        graph, static_out, shim_bytes, allocations = _capture(device, lambda: ffn_shim(static_x, None, DECODE))
        assert allocations == capture_allocations + 1  # the output tensor
        assert shim_bytes <= max(runtime_bytes, 0) + RUNTIME_SLACK_BYTES, (shim_bytes, runtime_bytes)
        _clean(transport)  # capture itself ran nothing

        for index, x in enumerate(inputs + inputs[:1]):
            static_x.copy_(to_device(x, device))
            torch.cuda.synchronize()
            free = torch.cuda.mem_get_info(device)[0]
            allocations = torch.cuda.memory_stats(device)["allocation.all.allocated"]
            graph.replay()
            torch.cuda.synchronize()
            assert torch.cuda.mem_get_info(device)[0] == free
            assert torch.cuda.memory_stats(device)["allocation.all.allocated"] == allocations
            _clean(transport)
            replayed = static_out.cpu()
            eager = ffn_shim(to_device(x, device), None, DECODE)  # eager work between replays
            torch.cuda.synchronize()
            _clean(transport)
            assert_bitwise_equal(replayed, eager.cpu())
            if index == 0:
                assert_ffn_parity(
                    replayed, o.dense_partial_reference(x, w_gate_up, w_down), o.dense_fp32(x, w_gate_up, w_down)
                )
        agent.check_health()
        del graph
    finally:
        detach()
        agent.close()
