"""Execution Signatures (GraphTemplate keys), capacity buckets and workspace geometry.

Mirrors src/xpool/runtime/ffnagent/execution.py for the Dense path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from crosspool_amd.ffn import GateTransform, SiluActivation

OPERATOR_ALIGNMENT_BYTES = 16  # execution.py:16


def align_up(value: int, alignment: int) -> int:
    return (value + alignment - 1) // alignment * alignment


@dataclass(frozen=True, slots=True)
class WorkspaceLayout:
    """Prepared byte regions borrowed from one caller-owned backing (execution.py:38-70)."""

    regions: tuple[tuple[torch.dtype, tuple[int, ...]], ...]
    offsets: tuple[int, ...]
    nbytes: int

    @classmethod
    def from_regions(cls, regions: tuple[tuple[torch.dtype, tuple[int, ...]], ...]) -> WorkspaceLayout:
        """Align every non-empty region to 16 bytes, in order (execution.py:46-58)."""

        offsets = []
        cursor = 0
        for dtype, shape in regions:
            size = math.prod(shape) * dtype.itemsize
            if size:
                cursor = align_up(cursor, OPERATOR_ALIGNMENT_BYTES)
            offsets.append(cursor)
            cursor += size
        return cls(regions=regions, offsets=tuple(offsets), nbytes=cursor)

    def views(self, backing: torch.Tensor) -> tuple[torch.Tensor, ...]:
        """Borrow the prepared views without allocating (execution.py:60-70)."""

        if backing.dtype is not torch.uint8 or backing.ndim != 1 or not backing.is_contiguous():
            raise ValueError("workspace backing must be a contiguous byte vector")
        if backing.numel() < self.nbytes or backing.data_ptr() % OPERATOR_ALIGNMENT_BYTES:
            raise ValueError("workspace backing does not cover its prepared aligned extent")
        return tuple(
            backing[offset : offset + math.prod(shape) * dtype.itemsize].view(dtype).view(shape)
            for offset, (dtype, shape) in zip(self.offsets, self.regions, strict=True)
        )


def derive_payload_row_capacities(maximum_row_capacity: int) -> tuple[int, ...]:
    """Increasing power-of-two capacities through one exact maximum (execution.py:166-177)."""

    if isinstance(maximum_row_capacity, bool) or not isinstance(maximum_row_capacity, int):
        raise TypeError("maximum payload row capacity must be an integer")
    if maximum_row_capacity <= 0:
        raise ValueError("maximum payload row capacity must be positive")
    capacities = []
    capacity = 1
    while capacity < maximum_row_capacity:
        capacities.append(capacity)
        capacity *= 2
    capacities.append(maximum_row_capacity)
    return tuple(capacities)


def select_capacity(capacities: tuple[int, ...], rows: int) -> int:
    """Smallest installed capacity containing ``rows`` (src/cext/ffnagent/runtime.cu:246-253).

    The native replay applies the same rule; this host copy serves planning
    and error messages.
    """

    for capacity in sorted(capacities):
        if rows <= capacity:
            return capacity
    raise ValueError(f"{rows} rows exceed the largest installed capacity {max(capacities, default=0)}")


@dataclass(frozen=True, slots=True)
class DenseFfnExecutionSignature:
    """Complete reusable Dense graph identity (execution.py:73-95).

    One GraphTemplate is captured per signature and Lane; layers with equal
    signatures share it and differ only in their bound weights.
    """

    payload_dtype: torch.dtype
    payload_row_capacity: int
    hidden_size: int
    local_intermediate_size: int
    activation: SiluActivation = SiluActivation()
    gate: GateTransform = GateTransform()

    def __post_init__(self) -> None:
        if self.payload_dtype is not torch.bfloat16:
            raise ValueError("the MI355X Dense path executes bf16 payloads")
        for name in ("payload_row_capacity", "hidden_size", "local_intermediate_size"):
            value = getattr(self, name)
            if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
                raise ValueError(f"{name} must be a positive integer")
        if self.hidden_size % 8 or self.local_intermediate_size % 8:
            raise ValueError("hidden and intermediate sizes must be multiples of 8 (16-byte rows)")
        if self.activation != SiluActivation() or self.gate != GateTransform():
            raise ValueError("captured Dense templates use the default SiLU gate (alpha 1, no limit, no offset)")

    @property
    def payload_shape(self) -> tuple[int, int]:
        return self.payload_row_capacity, self.hidden_size

    def workspace_layout(self) -> WorkspaceLayout:
        """Gathered batch then activated intermediate, both payload dtype."""

        return WorkspaceLayout.from_regions(
            (
                (self.payload_dtype, (self.payload_row_capacity, self.hidden_size)),
                (self.payload_dtype, (self.payload_row_capacity, self.local_intermediate_size)),
            )
        )


def dense_signatures(
    *, hidden_size: int, local_intermediate_size: int, maximum_row_capacity: int
) -> tuple[DenseFfnExecutionSignature, ...]:
    """Specialise one Dense layer layout over the capacity domain (preparation.py:38-55)."""

    return tuple(
        DenseFfnExecutionSignature(
            payload_dtype=torch.bfloat16,
            payload_row_capacity=capacity,
            hidden_size=hidden_size,
            local_intermediate_size=local_intermediate_size,
        )
        for capacity in derive_payload_row_capacities(maximum_row_capacity)
    )
