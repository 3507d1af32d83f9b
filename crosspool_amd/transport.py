"""Request metadata of one FFN shim call (mirrors src/xpool/transport.py:16-42)."""

from __future__ import annotations

from dataclasses import dataclass

from crosspool_amd.ffn import DpRowLayout, ForwardMode, OutputRequirement

__all__ = ["FfnRequestMetadata"]


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
