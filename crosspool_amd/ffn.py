"""Closed FFN vocabulary and the Dense activation semantics.

Mirrors ``xpool.native.ffn`` (values of src/cext-include/xpool/ffn.hpp:15-54)
and the activation / Gate-Up declarations of src/xpool/ffn.py:43-137.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum


class ForwardMode(IntEnum):
    """Runtime forward mode of one FFN request (ffn.hpp:15-22)."""

    PREFILL = 1
    DECODE = 2
    IDLE = 4


class OutputRequirement(IntEnum):
    """Mathematical output requirement (ffn.hpp:24-30)."""

    PER_RANK_COMPLETE = 1
    GROUP_SUM_COMPLETE = 2


class DpRowLayout(IntEnum):
    """Physical data-parallel row layout (ffn.hpp:32-40)."""

    NONE = 0
    UNIFORM_BY_RANK = 1
    PACKED_BY_RANK = 2


class ResultCode(IntEnum):
    """Completion result code (ffn.hpp:42-48)."""

    OK = 0
    SHUTDOWN = 1
    PROTOCOL_MISMATCH = 2
    TIMEOUT = 3


class LayerKind(IntEnum):
    """Structural kind of one gated FFN layer (ffn.hpp:50-54)."""

    DENSE = 1
    MOE = 2


class RouterAlgorithm(IntEnum):
    """Activated scoring rule of a MoE Router (src/xpool/ffn.py:78-82)."""

    SOFTMAX = 1
    SIGMOID = 2


class RouterProjectionPrecision(IntEnum):
    """Router projection input / weight / logits dtypes (src/xpool/ffn.py:85-102).

    PAYLOAD: bf16 weights and bf16 logits; FP32: fp32 weights over the widened input, fp32
    logits; FP32_LOGITS: bf16 weights, fp32 logits.
    """

    PAYLOAD = 1
    FP32 = 2
    FP32_LOGITS = 3


class TopKWeightRounding(IntEnum):
    """Extra rounding of routed mixing weights to the logits dtype (src/xpool/ffn.py:105-115)."""

    NONE = 1
    LOGITS_DTYPE = 2


class ActivationKind(IntEnum):
    """FFN activation semantics (src/xpool/ffn.py:43-48)."""

    SILU = 1
    RELU = 2
    GELU = 3


class GateUpOrder(IntEnum):
    """Physical ordering of the gate and up projection rows (src/xpool/ffn.py:51-68)."""

    CONCATENATED = 1
    INTERLEAVED = 2

    def row_indices(self, *, width: int, start: int, length: int) -> tuple[slice, slice]:
        """Gate then Up row selections of a prepared i_proj of intermediate ``width``."""

        if self is GateUpOrder.CONCATENATED:
            return slice(start, start + length), slice(width + start, width + start + length)
        return slice(2 * start, 2 * (start + length), 2), slice(2 * start + 1, 2 * (start + length), 2)


@dataclass(frozen=True)
class SiluActivation:
    """``x * sigmoid(alpha * x)`` (src/xpool/ffn.py:123-127)."""

    alpha: float = 1.0

    def __post_init__(self) -> None:
        if not (self.alpha > 0 and self.alpha != float("inf")):
            raise ValueError("SiLU alpha must be positive and finite")

    kind = ActivationKind.SILU


@dataclass(frozen=True)
class ReluActivation:
    """ReLU of one projection, NaN payloads kept (src/xpool/ffn.py:140-143)."""

    kind = ActivationKind.RELU


@dataclass(frozen=True)
class GeluActivation:
    """GELU with the erf definition (``"none"``) or the tanh approximation (ffn.py:146-150)."""

    approximate: str = "none"

    def __post_init__(self) -> None:
        if self.approximate not in ("none", "tanh"):
            raise ValueError("GELU approximation must be 'none' or 'tanh'")

    kind = ActivationKind.GELU


@dataclass(frozen=True)
class GateTransform:
    """Clip Gate above ``limit``, Up to ``[-limit, limit]``, then add ``up_offset`` (ffn.py:130-137)."""

    limit: float | None = None
    up_offset: float = 0.0

    def __post_init__(self) -> None:
        if self.limit is not None and not self.limit > 0:
            raise ValueError("gate limit must be positive")


def activation_arguments(activation: SiluActivation, gate: GateTransform) -> tuple[float, float, float]:
    """(alpha, limit or 0, up_offset) as the C ABI takes them."""

    return float(activation.alpha), float(gate.limit or 0.0), float(gate.up_offset)
