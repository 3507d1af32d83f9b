"""Request metadata of one FFN shim call and the Transport mailbox resident.

``FfnRequestMetadata`` mirrors src/xpool/transport.py:16-42; ``TransportResident`` is the
host side of the request mailboxes (src/cext/transport/, over the C ABI's xp_transport_*).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from enum import IntEnum

import torch

from crosspool_amd import _native
from crosspool_amd.ffn import DpRowLayout, ForwardMode, OutputRequirement, ResultCode

__all__ = ["ArenaSnapshot", "FfnRequestMetadata", "MailboxStatus", "TransportResident"]


@dataclass(frozen=True, slots=True)
class FfnRequestMetadata:
    """Transport wire metadata for one public FFN shim call.

    Attributes:
        layer_ordinal: Zero-based FFN position in the workload.
        forward_mode: Prefill, decode, or idle ABI value.
        output_requirement: Mathematical output requirement.
        dp_row_layout: Physical data-parallel row layout selected by the producer.
    """

    layer_ordinal: int
    forward_mode: ForwardMode
    output_requirement: OutputRequirement
    dp_row_layout: DpRowLayout

    def __post_init__(self) -> None:
        """Reject untyped request metadata before dispatch (transport.py:32-42)."""

        if isinstance(self.layer_ordinal, bool) or not isinstance(self.layer_ordinal, int) or self.layer_ordinal < 0:
            raise ValueError("xpool FFN layer ordinal must be a non-negative integer")
        if not isinstance(self.forward_mode, ForwardMode):
            raise TypeError("xpool FFN forward mode must be ForwardMode")
        if not isinstance(self.output_requirement, OutputRequirement):
            raise TypeError("xpool FFN output requirement must be OutputRequirement")
        if not isinstance(self.dp_row_layout, DpRowLayout):
            raise TypeError("xpool FFN DP row layout must be DpRowLayout")


class MailboxStatus(IntEnum):
    """Lifecycle of one request mailbox (src/cext-include/xpool/transport/protocol.hpp:33-49)."""

    DORMANT = 0
    IDLE = 1
    STAGING = 2
    PUBLISHED = 3
    EVALUATED = 4
    CLOSED = 5


class _Snapshot(ctypes.Structure):
    _fields_ = [
        ("mailbox_status", ctypes.c_uint32),
        ("result_code", ctypes.c_uint32),
        ("payload_rows", ctypes.c_uint64),
        ("layer_ordinal", ctypes.c_uint64),
        ("forward_mode", ctypes.c_uint32),
        ("output_requirement", ctypes.c_uint32),
        ("dp_row_layout", ctypes.c_uint32),
        ("shutdown", ctypes.c_uint32),
        ("generation_failure", ctypes.c_uint32),
        ("violations", ctypes.c_uint32),
        ("instance_outcome", ctypes.c_uint32),
        ("atn_dp_size", ctypes.c_uint32),
        ("payload_row_capacity", ctypes.c_uint64),
        ("dp_rank_payload_rows", ctypes.c_uint32 * 64),
    ]


@dataclass(frozen=True)
class ArenaSnapshot:
    """Host copy of one arena (Arena::state / mailbox_status of transport/arena.hpp).

    ``violations`` counts protocol preconditions found broken on the device (the reference
    traps on them); ``instance_outcome`` is the last completed request's result, or
    ``None`` while a request is between submit and complete.
    """

    mailbox_status: MailboxStatus
    result_code: int
    payload_rows: int
    request: tuple[int, int, int, int]
    shutdown: bool
    generation_failure: ResultCode
    violations: int
    instance_outcome: ResultCode | None
    atn_dp_size: int
    payload_row_capacity: int
    dp_rank_payload_rows: tuple[int, ...]


def _completion_output(output: torch.Tensor | None) -> tuple[ctypes.c_void_p | None, int, int]:
    """Pointer, element count and payload dtype code of a completion's output (bf16 or fp16)."""

    if output is None:
        return None, 0, _native.XP_DTYPE_BF16
    if output.dtype not in (torch.bfloat16, torch.float16) or not output.is_contiguous():
        raise ValueError("the completion output must be a contiguous bf16 or fp16 tensor")
    return ctypes.c_void_p(output.data_ptr()), output.numel(), _native.payload_dtype_code(output.dtype)


class TransportResident:
    """The Transport arenas of one device and the agent that answers their mailboxes.

    Mirrors the AtnAgent-owned arenas and TransportResident of
    src/cext/transport/atnagent.cpp / atnagent.cu: one arena (one SPSC mailbox) per
    Instance rank, opened together at startup and drained together.  On one GPU the
    Resident's polling loop becomes stream-ordered calls: :meth:`submit` and
    :meth:`complete` are the Instance kernel's two halves (instance.cu:36-201) on the
    caller's stream, :meth:`evaluate` answers a published request after the Dense step
    (on a Lane's stream, between two events), and :meth:`settle` does both answer and
    completion in one launch when the Dense step ran on the caller's stream.
    """

    def __init__(self, device: torch.device, arenas: list[tuple[int, int]]) -> None:
        """``arenas``: (payload_row_capacity, atn_dp_size) per Instance rank."""

        if not arenas:
            raise ValueError("a transport needs at least one arena")
        self.device = torch.device(device)
        self.layouts = tuple((int(c), int(d)) for c, d in arenas)
        capacities = (ctypes.c_int64 * len(arenas))(*(c for c, _ in self.layouts))
        dp_sizes = (ctypes.c_int32 * len(arenas))(*(d for _, d in self.layouts))
        handle = ctypes.c_void_p()
        _native.call(
            "xp_transport_create", self.device.index, len(arenas), capacities, dp_sizes, ctypes.byref(handle)
        )
        self.handle = handle

    def _stream(self, stream: torch.cuda.Stream | None) -> ctypes.c_void_p:
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        return ctypes.c_void_p(stream.cuda_stream)

    def _require_open(self) -> None:
        if self.handle is None:
            raise RuntimeError("Transport resident is closed")

    def open(self, stream: torch.cuda.Stream | None = None) -> None:
        """Resident startup: every Dormant mailbox becomes Idle (atnagent.cu:124-129)."""

        self._require_open()
        _native.call("xp_transport_open", self.handle, self._stream(stream))

    def submit(
        self,
        arena: int,
        payload_rows: int,
        request: FfnRequestMetadata,
        dp_rank_payload_rows: torch.Tensor | None = None,
        stream: torch.cuda.Stream | None = None,
    ) -> None:
        """Instance claim, staging and publication (instance.cu:46-128)."""

        self._require_open()
        present = dp_rank_payload_rows is not None and dp_rank_payload_rows.numel() != 0
        pointer = ctypes.c_void_p(dp_rank_payload_rows.data_ptr()) if present else None
        count = dp_rank_payload_rows.numel() if present else 0
        is_i64 = int(present and dp_rank_payload_rows.dtype is torch.int64)
        _native.call(
            "xp_transport_submit", self.handle, arena, payload_rows, request.layer_ordinal, int(request.forward_mode),
            int(request.output_requirement), int(request.dp_row_layout), pointer, count, is_i64, self._stream(stream),
        )

    def evaluate(self, arena: int, fault_word: int | None = None, stream: torch.cuda.Stream | None = None) -> None:
        """Answer a published request after the Dense step (atnagent.cu:48-90)."""

        self._require_open()
        fault = ctypes.c_void_p(fault_word) if fault_word else None
        _native.call("xp_transport_evaluate", self.handle, arena, fault, self._stream(stream))

    def complete(
        self,
        arena: int,
        output: torch.Tensor | None,
        *,
        timeout_ns: int = 0,
        stream: torch.cuda.Stream | None = None,
    ) -> None:
        """Observe the result; acknowledge, or close and NaN-fill ``output`` with quiet NaNs of its
        dtype (instance.cu:130-201)."""

        self._require_open()
        pointer, elements, dtype = _completion_output(output)
        _native.call("xp_transport_complete", self.handle, arena, pointer, elements, dtype, int(timeout_ns),
                     self._stream(stream))

    def settle(
        self,
        arena: int,
        output: torch.Tensor | None,
        fault_word: int | None = None,
        stream: torch.cuda.Stream | None = None,
    ) -> None:
        """:meth:`evaluate` then :meth:`complete` in one launch, after a Dense step on the same stream."""

        self._require_open()
        pointer, elements, dtype = _completion_output(output)
        fault = ctypes.c_void_p(fault_word) if fault_word else None
        _native.call("xp_transport_settle", self.handle, arena, fault, pointer, elements, dtype, self._stream(stream))

    def drain(self, stream: torch.cuda.Stream | None = None) -> None:
        """Publish shutdown to every arena and finish their mailboxes (atnagent.cu:92-147)."""

        self._require_open()
        _native.call("xp_transport_drain", self.handle, self._stream(stream))

    def publish_failure(self, arena: int, result: ResultCode, stream: torch.cuda.Stream | None = None) -> None:
        """Publish a canonical failure; the first one sticks (arena.cuh:55-62)."""

        self._require_open()
        _native.call("xp_transport_publish_failure", self.handle, arena, int(result), self._stream(stream))

    def snapshot(self, arena: int) -> ArenaSnapshot:
        """Synchronous host copy of one arena (waits for the device)."""

        self._require_open()
        raw = _Snapshot()
        _native.call("xp_transport_snapshot", self.handle, arena, ctypes.byref(raw))
        outcome = None if raw.instance_outcome == 0xFFFFFFFF else ResultCode(raw.instance_outcome)
        return ArenaSnapshot(
            mailbox_status=MailboxStatus(raw.mailbox_status),
            result_code=int(raw.result_code),
            payload_rows=int(raw.payload_rows),
            request=(int(raw.layer_ordinal), int(raw.forward_mode), int(raw.output_requirement), int(raw.dp_row_layout)),
            shutdown=bool(raw.shutdown),
            generation_failure=ResultCode(raw.generation_failure),
            violations=int(raw.violations),
            instance_outcome=outcome,
            atn_dp_size=int(raw.atn_dp_size),
            payload_row_capacity=int(raw.payload_row_capacity),
            dp_rank_payload_rows=tuple(int(v) for v in raw.dp_rank_payload_rows[: raw.atn_dp_size]),
        )

    def probe(self, arena: int, scenario: int) -> list[int]:
        """Run one of the reference's device-side protocol scenarios; its observation words."""

        self._require_open()
        words = (ctypes.c_uint32 * 16)()
        _native.call("xp_transport_probe", self.handle, arena, scenario, words, 16)
        return [int(w) for w in words]

    def close(self) -> None:
        if self.handle is not None:
            _native.call("xp_transport_destroy", self.handle)
            self.handle = None

    def __enter__(self) -> TransportResident:
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()
