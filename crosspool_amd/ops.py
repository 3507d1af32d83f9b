"""The ``ffn_shim`` Tensor operator: the SGLang-facing drop-in boundary.

Mirrors ``xpool.ops.ffn_shim`` (src/xpool/ops.py:15-53) and the synchronous
checks of ``InstanceRankRuntime::Attachment::submit``
(src/cext/transport/instance.cpp:82-123).  In this single-GPU build the
attachment is an in-process :class:`~crosspool_amd.agent.FfnAgent`: the
caller's hidden states are the mailbox and rows ``0..T-1`` are its slots, which
is exactly the reference's contiguous row-prefix Transport copy.

By default each call runs the reference's Transport mailbox transaction
(instance.cu:36-201, atnagent.cu:48-90) around the Dense step, all on the
caller's stream: the request is claimed and published, the Lane's kernels run the
step, and one launch answers the request and completes it (acknowledge, or the
NaN-filled canonical failure output).  With ``lane_stream=True`` the step and the
answer run on the Lane's own stream between two events instead (two cross-stream
hops, ~35 us more per call on MI355X).  ``attach(..., mailbox=False)`` runs the
step on the caller's stream without the mailbox.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass

import torch

from crosspool_amd.agent import FfnAgent
from crosspool_amd.ffn import DpRowLayout
from crosspool_amd.transport import FfnRequestMetadata, TransportResident

__all__ = ["attach", "attached_transport", "detach", "ffn_shim"]


@dataclass
class _Attachment:
    agent: FfnAgent
    instance_index: int
    hidden_size: int
    payload_dtype: torch.dtype
    capacity: int
    atn_dp_size: int
    lane: int
    identity_slots: torch.Tensor
    transport: TransportResident | None
    timeout_ns: int
    lane_stream: bool


_lock = threading.Lock()
_attachment: _Attachment | None = None


def attach(
    agent: FfnAgent,
    *,
    instance_index: int = 0,
    atn_dp_size: int = 1,
    lane: int = 0,
    mailbox: bool = True,
    lane_stream: bool = False,
    timeout_ns: int = 0,
) -> None:
    """Attach this process's shim to a materialized agent (Attachment::attach analogue).

    With ``mailbox`` a one-arena :class:`TransportResident` is created and opened, and
    every call runs the mailbox transaction, with the Dense step on the caller's stream
    or, with ``lane_stream``, on the Lane's stream; ``timeout_ns`` bounds the two-stream
    completion's wait (0: the reference's 5 s).
    """

    global _attachment
    if not agent.materialized:
        raise RuntimeError("attach requires a materialized FfnAgent")
    shapes = {(b.weights.hidden_size, b.payload_dtype) for (i, _), b in agent.layers.items() if i == instance_index}
    if len(shapes) != 1:
        raise ValueError("the attached instance must have registered layers of one hidden size and payload dtype")
    hidden_size, payload_dtype = shapes.pop()
    capacity = max(t.signature.payload_row_capacity for t in agent.templates.values())
    transport = None
    if mailbox:
        transport = TransportResident(agent.device, [(capacity, atn_dp_size)])
        transport.open()
    with _lock:
        previous = _attachment
        _attachment = _Attachment(
            agent=agent,
            instance_index=instance_index,
            hidden_size=hidden_size,
            payload_dtype=payload_dtype,
            capacity=capacity,
            atn_dp_size=atn_dp_size,
            lane=lane,
            identity_slots=torch.arange(capacity, dtype=torch.int32, device=agent.device),
            transport=transport,
            timeout_ns=int(timeout_ns),
            lane_stream=bool(lane_stream),
        )
    if previous is not None and previous.transport is not None:
        previous.transport.close()


def detach() -> None:
    """Drop the attachment; its Transport is drained and released."""

    global _attachment
    with _lock:
        previous = _attachment
        _attachment = None
    if previous is not None and previous.transport is not None:
        previous.transport.drain()
        previous.transport.close()


def attached_transport() -> TransportResident | None:
    """The attachment's Transport resident (``None`` without a mailbox)."""

    attachment = _attachment
    return None if attachment is None else attachment.transport


def ffn_shim(
    hidden_states: torch.Tensor,
    dp_rank_payload_rows: torch.Tensor | None,
    request_metadata: FfnRequestMetadata,
) -> torch.Tensor:
    """Dispatch one FFN request through the attached native execution.

    Args:
        hidden_states: Contiguous device tensor ``[payload_rows, hidden_size]``.
        dp_rank_payload_rows: Optional device int32/int64 vector, one physical
            row span per attention DP rank (required iff ``atn_dp_size > 1``).
        request_metadata: Validated transport metadata for this invocation.

    Returns:
        Tensor with the same shape, dtype and device as ``hidden_states``.

    Raises:
        RuntimeError: If nothing is attached, rows exceed the installed
            capacity, or the tensor contract is violated (instance.cpp:91-119).

    Side effects:
        Stream-ordered on the current stream; never synchronises the host.
    """

    attachment = _attachment
    if attachment is None:
        raise RuntimeError("xpool FFN shim has no attached FfnAgent")
    if not isinstance(request_metadata, FfnRequestMetadata):
        raise RuntimeError("xpool FFN shim received invalid request metadata")
    if hidden_states.dim() != 2:
        raise RuntimeError("xpool FFN shim expects a 2D hidden-state tensor")
    payload_rows = hidden_states.shape[0]
    present = dp_rank_payload_rows is not None and dp_rank_payload_rows.numel() != 0
    if not 0 < payload_rows <= attachment.capacity:
        raise RuntimeError("xpool FFN request row count exceeds Transport capacity")
    if attachment.atn_dp_size == 1:
        if request_metadata.dp_row_layout is not DpRowLayout.NONE or present:
            raise RuntimeError("xpool DP-one request must use NONE without a per-rank row vector")
    else:
        if request_metadata.dp_row_layout not in (DpRowLayout.UNIFORM_BY_RANK, DpRowLayout.PACKED_BY_RANK):
            raise RuntimeError("xpool DP request requires UNIFORM_BY_RANK or PACKED_BY_RANK")
        if not present:
            raise RuntimeError("xpool DP request requires one physical row value per attention DP rank")
        if dp_rank_payload_rows.numel() != attachment.atn_dp_size:
            raise RuntimeError("xpool FFN shim DP-rank payload rows must have one entry per attention DP rank")
        if dp_rank_payload_rows.dtype not in (torch.int32, torch.int64) or dp_rank_payload_rows.device != hidden_states.device:
            raise RuntimeError("xpool FFN shim DP-rank payload rows must be a device int32 or int64 tensor")
    if hidden_states.shape[1] != attachment.hidden_size:
        raise RuntimeError("xpool FFN shim hidden size does not match the attached Transport arena")
    if hidden_states.dtype is not attachment.payload_dtype:
        raise RuntimeError("xpool FFN shim dtype does not match the attached Transport arena")
    if hidden_states.device != attachment.agent.device:
        raise RuntimeError("xpool FFN shim hidden states must be on the attached Transport arena device")
    if not hidden_states.is_contiguous():
        raise RuntimeError("xpool FFN shim hidden states must be contiguous")
    if (attachment.instance_index, request_metadata.layer_ordinal) not in attachment.agent.layers:
        raise RuntimeError(f"xpool FFN shim layer {request_metadata.layer_ordinal} is not installed")

    output = torch.empty_like(hidden_states)
    agent = attachment.agent
    caller = torch.cuda.current_stream(hidden_states.device)
    transport = attachment.transport
    # The FFN is row-independent, so every DP row layout is served by running
    # all physical rows; padding rows of UNIFORM_BY_RANK spans compute garbage
    # that the producer never reads.
    if transport is None:
        agent.execute(
            instance_index=attachment.instance_index,
            layer_ordinal=request_metadata.layer_ordinal,
            pool=hidden_states,
            out_pool=output,
            slots=attachment.identity_slots,
            rows=payload_rows,
            lane=attachment.lane,
            stream=caller,
        )
        return output
    lane = agent.lanes[attachment.lane]
    rows_vector = dp_rank_payload_rows if present else None
    transport.submit(0, payload_rows, request_metadata, rows_vector, stream=caller)
    if not attachment.lane_stream:
        agent.execute(
            instance_index=attachment.instance_index,
            layer_ordinal=request_metadata.layer_ordinal,
            pool=hidden_states,
            out_pool=output,
            slots=attachment.identity_slots,
            rows=payload_rows,
            lane=attachment.lane,
            stream=caller,
        )
        transport.settle(0, output, lane.fault_word, stream=caller)
        return output
    # The Lane stream waits for the published request, runs the Dense step and answers it.
    agent.execute(
        instance_index=attachment.instance_index,
        layer_ordinal=request_metadata.layer_ordinal,
        pool=hidden_states,
        out_pool=output,
        slots=attachment.identity_slots,
        rows=payload_rows,
        lane=attachment.lane,
    )
    transport.evaluate(0, lane.fault_word, stream=lane.stream)
    caller.wait_stream(lane.stream)
    transport.complete(0, output, timeout_ns=attachment.timeout_ns, stream=caller)
    return output
