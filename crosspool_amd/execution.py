"""Execution Signatures (GraphTemplate keys), capacity buckets and workspace geometry.

Mirrors src/xpool/runtime/ffnagent/execution.py for the Dense and MoE layer kinds.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from crosspool_amd.ffn import (
    GateTransform,
    GeluActivation,
    ReluActivation,
    RouterAlgorithm,
    RouterProjectionPrecision,
    SiluActivation,
    TopKWeightRounding,
    activation_arguments,
)

OPERATOR_ALIGNMENT_BYTES = 16  # execution.py:16


def align_up(value: int, alignment: int) -> int:
    return (value + alignment - 1) // alignment * alignment


@dataclass(frozen=True, slots=True)
class WorkspaceLayout:
    """Typed regions placed one after another in a caller-owned byte buffer.

    The placement rule is the reference's (execution.py:38-70, pinned by its known answers):
    regions keep their order, and each non-empty region starts at the next multiple of
    OPERATOR_ALIGNMENT_BYTES; an empty region takes the current offset and no space.
    """

    regions: tuple[tuple[torch.dtype, tuple[int, ...]], ...]
    offsets: tuple[int, ...]
    nbytes: int

    @staticmethod
    def region_bytes(region: tuple[torch.dtype, tuple[int, ...]]) -> int:
        dtype, shape = region
        return dtype.itemsize * math.prod(shape)

    @classmethod
    def from_regions(cls, regions: tuple[tuple[torch.dtype, tuple[int, ...]], ...]) -> WorkspaceLayout:
        placed: list[int] = []
        end = 0
        for region in regions:
            size = cls.region_bytes(region)
            start = align_up(end, OPERATOR_ALIGNMENT_BYTES) if size else end
            placed.append(start)
            end = start + size
        return cls(regions=regions, offsets=tuple(placed), nbytes=end)

    def views(self, backing: torch.Tensor) -> tuple[torch.Tensor, ...]:
        """One typed view per region into ``backing`` (a flat uint8 tensor); nothing is allocated."""

        flat_bytes = backing.dtype is torch.uint8 and backing.dim() == 1 and backing.is_contiguous()
        if not flat_bytes:
            raise ValueError(f"a workspace is a flat contiguous uint8 tensor, not {backing.dtype} {tuple(backing.shape)}")
        if backing.data_ptr() % OPERATOR_ALIGNMENT_BYTES:
            raise ValueError(f"a workspace must start on a {OPERATOR_ALIGNMENT_BYTES}-byte boundary")
        if backing.numel() < self.nbytes:
            raise ValueError(f"workspace holds {backing.numel()} bytes; this layout needs {self.nbytes}")
        views = []
        for offset, region in zip(self.offsets, self.regions):
            dtype, shape = region
            views.append(backing.narrow(0, offset, self.region_bytes(region)).view(dtype).reshape(shape))
        return tuple(views)


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
        if self.payload_dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("the MI355X Dense path executes bf16 or fp16 payloads (ffn.hpp:83-85)")
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


@dataclass(frozen=True, slots=True)
class MoeRouterExecutionSignature:
    """Router-owner part of a MoE graph identity (execution.py:98-108).

    On one device the Lane always owns the Router.  Whether a correction bias is bound does
    not change the captured body (the bias is an argument of the TopK kernel), so it is not
    part of the identity here.
    """

    algorithm: RouterAlgorithm
    projection_precision: RouterProjectionPrecision
    weight_rounding: TopKWeightRounding
    routed_expert_count: int
    routed_topk: int
    renormalize: bool


@dataclass(frozen=True, slots=True)
class MoeFfnExecutionSignature:
    """Complete reusable MoE graph identity (execution.py:111-149)."""

    payload_dtype: torch.dtype
    payload_row_capacity: int
    hidden_size: int
    local_intermediate_size: int
    expert_count: int
    effective_topk: int
    routed_scaling_factor: float
    router: MoeRouterExecutionSignature
    activation: SiluActivation | ReluActivation | GeluActivation = SiluActivation()
    gate: GateTransform = GateTransform()
    # Projection biases of the layer's experts (ProjectionLayout.bias): bit 0 i_proj, bit 1 o_proj.
    biases: int = 0

    def __post_init__(self) -> None:
        if self.payload_dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("MoE payloads must be bf16 or fp16")
        for name in ("payload_row_capacity", "hidden_size", "local_intermediate_size", "expert_count", "effective_topk"):
            value = getattr(self, name)
            if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
                raise ValueError(f"{name} must be a positive integer")
        shared = self.expert_count - self.router.routed_expert_count
        if shared < 0 or self.effective_topk != self.router.routed_topk + shared:
            raise ValueError("effective TopK must be the routed TopK plus the shared expert count")

    @property
    def payload_shape(self) -> tuple[int, int]:
        return self.payload_row_capacity, self.hidden_size

    @property
    def routing_shape(self) -> tuple[int, int]:
        """Route ids / weights geometry (execution.py:131-135)."""

        return self.payload_row_capacity, self.effective_topk

    @property
    def routing_storage_bytes(self) -> int:
        """Packed int32 ids and fp32 weights (execution.py:137-141)."""

        return math.prod(self.routing_shape) * (torch.int32.itemsize + torch.float32.itemsize)

    def native_descriptor(self):
        """The ``xp_moe_layer_desc`` of this signature."""

        from crosspool_amd import _native

        silu = isinstance(self.activation, SiluActivation)
        alpha, limit, up_offset = activation_arguments(self.activation if silu else SiluActivation(), self.gate)
        router = self.router
        return _native.MoeLayerDesc(
            hidden=self.hidden_size,
            intermediate=self.local_intermediate_size,
            experts=self.expert_count,
            routed_experts=router.routed_expert_count,
            routed_topk=router.routed_topk,
            algorithm=int(router.algorithm),
            precision=int(router.projection_precision),
            renormalize=int(router.renormalize),
            weight_rounding=int(router.weight_rounding),
            routed_scaling_factor=float(self.routed_scaling_factor),
            alpha=alpha,
            limit=limit,
            up_offset=up_offset,
            payload=_native.payload_dtype_code(self.payload_dtype),
            activation=int(self.activation.kind),
            approximate_tanh=int(isinstance(self.activation, GeluActivation) and self.activation.approximate == "tanh"),
            biases=int(self.biases),
        )
