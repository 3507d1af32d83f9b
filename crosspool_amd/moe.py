"""MoE Router, routing finalisation and Experts over caller-owned storage.

Mirrors the reference operators (paths relative to the CrossPool checkout):

* ``Router`` / ``RouterExecutionPlan``: src/xpool/runtime/ffnagent/operators/routing.py:92-190;
* ``finalize_moe_routing``: routing.py:230-307;
* ``Experts`` / ``ExpertExecutionPlan``: src/xpool/runtime/ffnagent/operators/moe.py:112-343;
* ``MoeRouterWeights`` / ``MoeFfnWeights``: src/xpool/runtime/ffnagent/weights.py:171-230.

Every launch goes to the HIP library (``xp_moe_*``) on the current torch stream; nothing
here computes on the CPU.  Workspaces are allocated once per operator, so ``run_into``
allocates nothing.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from crosspool_amd import _native
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
from crosspool_amd.weights import validate_weight_tensor

__all__ = [
    "Experts",
    "MoeFfnWeights",
    "MoeLayerSpec",
    "MoeRouterWeights",
    "Router",
    "finalize_moe_routing",
]


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def _require(tensor: torch.Tensor, name: str, dtype: torch.dtype, shape: tuple[int, ...]) -> None:
    if tensor.device.type != "cuda" or tensor.dtype is not dtype or tuple(tensor.shape) != shape:
        raise ValueError(f"{name} must be a {dtype} GPU tensor of shape {shape}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


@dataclass(frozen=True, slots=True)
class MoeRouterWeights:
    """Router projection ``[experts, hidden]`` and optional fp32 selection-only correction (weights.py:171-187)."""

    projection: torch.Tensor
    correction_bias: torch.Tensor | None = None

    def __post_init__(self) -> None:
        validate_weight_tensor(self.projection, name="router projection")
        if self.projection.ndim != 2 or self.projection.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise ValueError("Router projection requires a bf16, fp16 or fp32 matrix")
        if self.correction_bias is not None:
            validate_weight_tensor(self.correction_bias, name="router correction bias")
            if self.correction_bias.dtype is not torch.float32 or self.correction_bias.ndim != 1:
                raise ValueError("Router correction bias requires a one-dimensional FP32 Tensor")
            if self.correction_bias.shape != self.projection.shape[:1]:
                raise ValueError("Router correction bias cardinality disagrees with its projection")
            if self.correction_bias.device != self.projection.device:
                raise ValueError("Router resources must share one device")


@dataclass(frozen=True, slots=True)
class MoeFfnWeights:
    """Expert projections and the optional Router (weights.py:190-230).

    ``i_proj`` is ``[experts, 2 I, H]`` with INTERLEAVED Gate/Up rows per expert,
    ``o_proj`` is ``[experts, H, I]``, both of the payload dtype (bf16 or fp16, the
    reference's supported payloads, src/cext-include/xpool/ffn.hpp:83-85).  The optional
    projection biases (``ProjectionWeights.bias``, weights.py:96-130) are fp32
    ``[experts, 2 I]`` (i_proj's row order) and ``[experts, H]``.
    """

    i_proj: torch.Tensor
    o_proj: torch.Tensor
    router: MoeRouterWeights | None = None
    i_proj_bias: torch.Tensor | None = None
    o_proj_bias: torch.Tensor | None = None

    def __post_init__(self) -> None:
        validate_weight_tensor(self.i_proj, name="Expert i_proj")
        validate_weight_tensor(self.o_proj, name="Expert o_proj")
        if self.i_proj.dtype not in (torch.bfloat16, torch.float16) or self.o_proj.dtype is not self.i_proj.dtype:
            raise ValueError("Expert projections must both be bf16 or both fp16")
        if self.i_proj.ndim != 3 or self.o_proj.ndim != 3:
            raise ValueError("Expert projections must be [experts, N, K] tensors")
        experts, two_i, hidden = self.i_proj.shape
        if tuple(self.o_proj.shape) != (experts, hidden, two_i // 2) or two_i % 2:
            raise ValueError("Expert projections disagree: i_proj [E, 2I, H] needs o_proj [E, H, I]")
        if self.i_proj.device != self.o_proj.device:
            raise ValueError("Expert projections must share one device")
        for bias, name, shape in (
            (self.i_proj_bias, "i_proj bias", (experts, two_i)),
            (self.o_proj_bias, "o_proj bias", (experts, hidden)),
        ):
            if bias is None:
                continue
            validate_weight_tensor(bias, name=f"Expert {name}")
            if bias.dtype is not torch.float32 or tuple(bias.shape) != shape:
                raise ValueError(f"Expert {name} must be an fp32 [{shape[0]}, {shape[1]}] tensor")
            if bias.device != self.i_proj.device:
                raise ValueError("Expert projections and biases must share one device")

    @property
    def expert_count(self) -> int:
        return int(self.i_proj.shape[0])

    @property
    def payload_dtype(self) -> torch.dtype:
        """The dtype of the layer's payloads: its expert projections'."""

        return self.i_proj.dtype

    @property
    def hidden_size(self) -> int:
        return int(self.i_proj.shape[2])

    @property
    def local_intermediate_size(self) -> int:
        return int(self.o_proj.shape[2])


@dataclass(frozen=True, slots=True)
class MoeLayerSpec:
    """Routing and activation declaration of one MoE layer.

    The fields of the reference's MoeFfnSpec (src/xpool/ffn.py:251-275) that execution
    reads, with the model-wide SiLU and GateTransform (ffn.py:346-356).  Experts
    ``[routed_expert_count, routed_expert_count + shared_expert_count)`` of the layer's
    weights are the always-selected shared ones.
    """

    routed_expert_count: int
    routed_topk: int
    shared_expert_count: int = 0
    renormalize: bool = True
    routed_scaling_factor: float = 1.0
    router_algorithm: RouterAlgorithm = RouterAlgorithm.SOFTMAX
    router_projection_precision: RouterProjectionPrecision = RouterProjectionPrecision.PAYLOAD
    topk_weight_rounding: TopKWeightRounding = TopKWeightRounding.NONE
    activation: SiluActivation | ReluActivation | GeluActivation = SiluActivation()
    gate: GateTransform = GateTransform()

    def __post_init__(self) -> None:
        if not 1 <= self.routed_topk <= min(self.routed_expert_count, 64):
            raise ValueError("routed TopK must be between 1 and min(routed experts, 64)")
        if self.shared_expert_count < 0 or self.routed_expert_count + self.shared_expert_count > 1024:
            raise ValueError("a MoE layer holds at most 1024 experts, shared ones included")
        if not (math.isfinite(self.routed_scaling_factor) and self.routed_scaling_factor > 0):
            raise ValueError("routed scaling factor must be finite and positive")

    @property
    def expert_count(self) -> int:
        return self.routed_expert_count + self.shared_expert_count

    @property
    def effective_topk(self) -> int:
        return self.routed_topk + self.shared_expert_count

    def validate_weights(self, weights: MoeFfnWeights) -> None:
        """Check a layer's resources against this declaration (registry.py:153-174)."""

        if weights.expert_count != self.expert_count:
            raise ValueError(
                f"MoE weights hold {weights.expert_count} experts; the layer declares {self.expert_count}"
            )
        if weights.router is None:
            raise ValueError("the Lane owns the Router on one device: MoE weights need a Router projection")
        weight_dtype = (
            torch.float32 if self.router_projection_precision is RouterProjectionPrecision.FP32
            else weights.payload_dtype
        )
        projection = weights.router.projection
        if projection.dtype is not weight_dtype or tuple(projection.shape) != (
            self.routed_expert_count, weights.hidden_size
        ):
            raise ValueError(
                f"router projection must be {weight_dtype} [{self.routed_expert_count}, {weights.hidden_size}]"
            )
        if weights.router.projection.device != weights.i_proj.device:
            raise ValueError("Router and Expert resources must share one device")

    def signature(
        self, *, hidden_size: int, local_intermediate_size: int, payload_row_capacity: int,
        payload_dtype: torch.dtype = torch.bfloat16, biases: int = 0,
    ):
        """The MoeFfnExecutionSignature of this layer at one capacity."""

        from crosspool_amd.execution import MoeFfnExecutionSignature, MoeRouterExecutionSignature

        return MoeFfnExecutionSignature(
            payload_dtype=payload_dtype,
            payload_row_capacity=payload_row_capacity,
            hidden_size=hidden_size,
            local_intermediate_size=local_intermediate_size,
            expert_count=self.expert_count,
            effective_topk=self.effective_topk,
            routed_scaling_factor=float(self.routed_scaling_factor),
            router=MoeRouterExecutionSignature(
                algorithm=RouterAlgorithm(self.router_algorithm),
                projection_precision=RouterProjectionPrecision(self.router_projection_precision),
                weight_rounding=TopKWeightRounding(self.topk_weight_rounding),
                routed_expert_count=self.routed_expert_count,
                routed_topk=self.routed_topk,
                renormalize=bool(self.renormalize),
            ),
            activation=self.activation,
            gate=self.gate,
            biases=biases,
        )


class Router:
    """Projection and TopK over a fixed row capacity (routing.py:92-190).

    ``ids`` ``[C, topk]`` int32 and ``weights`` ``[C, topk]`` fp32 are the outputs, written by
    :meth:`run_into` for the first ``rows`` rows (default: all ``C``).
    """

    def __init__(
        self,
        *,
        row_capacity: int,
        hidden_size: int,
        routed_expert_count: int,
        routed_topk: int,
        algorithm: RouterAlgorithm = RouterAlgorithm.SOFTMAX,
        precision: RouterProjectionPrecision = RouterProjectionPrecision.PAYLOAD,
        renormalize: bool = True,
        weight_rounding: TopKWeightRounding = TopKWeightRounding.NONE,
        device: torch.device | None = None,
        payload_dtype: torch.dtype = torch.bfloat16,
    ) -> None:
        if not 1 <= routed_topk <= min(routed_expert_count, 64) or routed_expert_count > 1024:
            raise ValueError("Router supports up to 1024 experts and a TopK of at most min(experts, 64)")
        if hidden_size <= 0:
            raise ValueError("hidden size must be positive")
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self.row_capacity = row_capacity
        self.hidden_size = hidden_size
        self.routed_expert_count = routed_expert_count
        self.routed_topk = routed_topk
        self.algorithm = RouterAlgorithm(algorithm)
        self.precision = RouterProjectionPrecision(precision)
        self.renormalize = bool(renormalize)
        self.weight_rounding = TopKWeightRounding(weight_rounding)
        self.payload_dtype = payload_dtype
        self._payload_code = _native.payload_dtype_code(payload_dtype)
        nbytes = _native.library().xp_moe_router_workspace_bytes(
            row_capacity, hidden_size, routed_expert_count, int(self.precision)
        )
        self.workspace = torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=self.device)
        self.ids = torch.empty((row_capacity, routed_topk), dtype=torch.int32, device=self.device)
        self.weights = torch.empty((row_capacity, routed_topk), dtype=torch.float32, device=self.device)
        logits_dtype = payload_dtype if self.precision is RouterProjectionPrecision.PAYLOAD else torch.float32
        count = row_capacity * routed_expert_count
        # The projection's logits, the first region of the workspace.
        self.logits = self.workspace[: count * logits_dtype.itemsize].view(logits_dtype).view(
            row_capacity, routed_expert_count
        )

    def run_into(self, *, hidden_states: torch.Tensor, router_weights: MoeRouterWeights, rows: int | None = None) -> None:
        rows = self.row_capacity if rows is None else rows
        if not 0 < rows <= self.row_capacity:
            raise ValueError("router rows must be positive and within the capacity")
        if hidden_states.dtype is not self.payload_dtype or hidden_states.shape[1:] != (self.hidden_size,):
            raise ValueError(f"router hidden states must be {self.payload_dtype} [rows, hidden]")
        if hidden_states.shape[0] < rows or not hidden_states.is_contiguous():
            raise ValueError("router hidden states must be contiguous and cover the rows")
        weight_dtype = torch.float32 if self.precision is RouterProjectionPrecision.FP32 else self.payload_dtype
        projection = router_weights.projection
        if projection.dtype is not weight_dtype or tuple(projection.shape) != (
            self.routed_expert_count, self.hidden_size
        ):
            raise ValueError(f"router projection must be {weight_dtype} [{self.routed_expert_count}, {self.hidden_size}]")
        _native.call(
            "xp_moe_router", _ptr(hidden_states), rows, self.hidden_size, _ptr(projection), self.routed_expert_count,
            self.routed_topk, int(self.algorithm), int(self.precision), self._payload_code,
            _ptr(router_weights.correction_bias),
            int(self.renormalize), int(self.weight_rounding), _ptr(self.ids), _ptr(self.weights),
            _ptr(self.workspace), self.workspace.numel(), _stream(),
        )


def router_topk(
    logits: torch.Tensor,
    *,
    topk: int,
    algorithm: RouterAlgorithm,
    correction_bias: torch.Tensor | None = None,
    renormalize: bool = True,
    weight_rounding: TopKWeightRounding = TopKWeightRounding.NONE,
    ids: torch.Tensor | None = None,
    weights: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """TopK alone over given bf16, fp16 or fp32 logits ``[rows, experts]`` (router_topk_kernel, routing.py:21-89)."""

    if logits.dtype not in (torch.bfloat16, torch.float16, torch.float32) or logits.ndim != 2 or not logits.is_contiguous():
        raise ValueError("logits must be a contiguous bf16, fp16 or fp32 matrix")
    rows, experts = logits.shape
    ids = torch.empty((rows, topk), dtype=torch.int32, device=logits.device) if ids is None else ids
    weights = torch.empty((rows, topk), dtype=torch.float32, device=logits.device) if weights is None else weights
    _require(ids, "ids", torch.int32, (rows, topk))
    _require(weights, "weights", torch.float32, (rows, topk))
    _native.call(
        "xp_moe_router_topk", _ptr(logits),
        _native.XP_DTYPE_F32 if logits.dtype is torch.float32 else _native.payload_dtype_code(logits.dtype),
        rows, experts, topk, int(algorithm),
        _ptr(correction_bias), int(renormalize), int(weight_rounding), _ptr(ids), _ptr(weights), _stream(),
    )
    return ids, weights


def finalize_moe_routing(
    *,
    routed_ids: torch.Tensor,
    routed_weights: torch.Tensor,
    final_ids: torch.Tensor,
    final_weights: torch.Tensor,
    payload_rows: torch.Tensor,
    routed_expert_count: int,
    shared_expert_count: int,
    routed_scaling_factor: float,
) -> None:
    """Fixed-capacity Routing Metadata in one kernel (routing.py:230-307, same checks)."""

    if routed_ids.dtype is not torch.int32 or routed_weights.dtype is not torch.float32:
        raise ValueError("routed Expert ids must be int32 and weights fp32")
    if routed_ids.ndim != 2 or routed_weights.shape != routed_ids.shape:
        raise ValueError("routed Expert id and weight dimensions disagree")
    row_capacity, routed_topk = routed_ids.shape
    effective_topk = routed_topk + shared_expert_count
    if final_ids.shape != (row_capacity, effective_topk) or final_weights.shape != final_ids.shape:
        raise ValueError("final Routing Metadata dimensions disagree")
    if final_ids.dtype is not torch.int32 or final_weights.dtype is not torch.float32:
        raise ValueError("final Expert ids must be int32 and weights fp32")
    if payload_rows.dtype is not torch.int64 or payload_rows.numel() != 1:
        raise ValueError("payload rows must contain exactly one int64 element")
    if routed_expert_count < routed_topk or shared_expert_count < 0:
        raise ValueError("Routing Metadata Expert counts are inconsistent")
    if not math.isfinite(routed_scaling_factor) or routed_scaling_factor <= 0:
        raise ValueError("routed scaling factor must be finite and positive")
    tensors = (routed_ids, routed_weights, final_ids, final_weights, payload_rows)
    if any(t.device != routed_ids.device or not t.is_contiguous() for t in tensors):
        raise ValueError("Routing Metadata tensors must share one device and be contiguous")
    if not torch.cuda.is_current_stream_capturing():
        live_rows = int(payload_rows.item())
        if live_rows <= 0 or live_rows > row_capacity:
            raise ValueError("payload rows must be positive and no greater than Capacity")
    _native.call(
        "xp_moe_finalize_routing", _ptr(routed_ids), _ptr(routed_weights), row_capacity, routed_topk,
        _ptr(final_ids), _ptr(final_weights), effective_topk, _ptr(payload_rows), routed_expert_count,
        float(routed_scaling_factor), _stream(),
    )


class Experts:
    """Grouped Expert FFN over a fixed row capacity (moe.py:112-343).

    ``run_into`` writes ``output[C, H] = scale * sum over each row's routes`` of the
    expert FFN of the row weighted by its route weight; ids of -1 are no route.
    """

    def __init__(
        self,
        *,
        row_capacity: int,
        hidden_size: int,
        local_intermediate_size: int,
        expert_count: int,
        effective_topk: int,
        routed_scaling_factor: float = 1.0,
        activation: SiluActivation | ReluActivation | GeluActivation | None = None,
        gate: GateTransform | None = None,
        device: torch.device | None = None,
        payload_dtype: torch.dtype = torch.bfloat16,
    ) -> None:
        if not math.isfinite(routed_scaling_factor) or routed_scaling_factor <= 0:
            raise ValueError("routed scaling factor must be finite and positive")
        if not 1 <= effective_topk <= expert_count <= 1024:
            raise ValueError("Experts support up to 1024 experts and a TopK within the expert count")
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        self.row_capacity = row_capacity
        self.hidden_size = hidden_size
        self.local_intermediate_size = local_intermediate_size
        self.expert_count = expert_count
        self.effective_topk = effective_topk
        self.routed_scaling_factor = float(routed_scaling_factor)
        activation = SiluActivation() if activation is None else activation
        if not isinstance(activation, (SiluActivation, ReluActivation, GeluActivation)):
            raise ValueError("Experts activation must be SiLU, ReLU or GELU")
        gate = GateTransform() if gate is None else gate
        alpha = float(activation.alpha) if isinstance(activation, SiluActivation) else 1.0
        _, limit, up_offset = activation_arguments(SiluActivation(alpha), gate)
        approximate = int(isinstance(activation, GeluActivation) and activation.approximate == "tanh")
        self.act = (int(activation.kind), approximate, alpha, limit, up_offset)
        self.payload_dtype = payload_dtype
        self._payload_code = _native.payload_dtype_code(payload_dtype)
        nbytes = _native.library().xp_moe_workspace_bytes(
            row_capacity, hidden_size, local_intermediate_size, expert_count, effective_topk
        )
        self.workspace = torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=self.device)

    def intermediates(self) -> dict[str, torch.Tensor]:
        """Views of the last call's workspace: the expert ends, sorted routes (route = row *
        topk + slot at each sorted position), activated routes (sorted order) and route
        outputs (by route).  Valid until the next :meth:`run_into`."""

        routes = self.row_capacity * self.effective_topk
        offsets = (ctypes.c_size_t * 6)()
        _native.call(
            "xp_moe_workspace_layout", self.row_capacity, self.hidden_size, self.local_intermediate_size,
            self.expert_count, self.effective_topk, offsets,
        )

        def view(index: int, dtype: torch.dtype, shape: tuple[int, ...]) -> torch.Tensor:
            count = math.prod(shape) * dtype.itemsize
            return self.workspace[offsets[index]: offsets[index] + count].view(dtype).view(shape)

        return {
            "expert_end": view(0, torch.int32, (self.expert_count,)),
            "sorted_route": view(1, torch.int32, (routes,)),
            "activated": view(4, self.payload_dtype, (routes, self.local_intermediate_size)),
            "route_out": view(5, self.payload_dtype, (routes, self.hidden_size)),
        }

    def run_into(
        self,
        *,
        hidden_states: torch.Tensor,
        weights: MoeFfnWeights,
        topk_ids: torch.Tensor,
        topk_weights: torch.Tensor,
        output: torch.Tensor,
    ) -> None:
        c, h, k = self.row_capacity, self.hidden_size, self.effective_topk
        _require(hidden_states, "hidden states", self.payload_dtype, (c, h))
        _require(output, "output", self.payload_dtype, (c, h))
        if weights.payload_dtype is not self.payload_dtype:
            raise ValueError(f"Expert weights must be {self.payload_dtype}")
        _require(topk_ids, "TopK ids", torch.int32, (c, k))
        _require(topk_weights, "TopK weights", torch.float32, (c, k))
        if (weights.expert_count, weights.hidden_size, weights.local_intermediate_size) != (
            self.expert_count, h, self.local_intermediate_size
        ):
            raise ValueError("Expert weights disagree with the operator geometry")
        function, approximate, alpha, limit, up_offset = self.act
        _native.call(
            "xp_moe_experts", _ptr(hidden_states), c, h, self.local_intermediate_size, self.expert_count, k,
            _ptr(weights.i_proj), _ptr(weights.o_proj), _ptr(weights.i_proj_bias), _ptr(weights.o_proj_bias),
            _ptr(topk_ids), _ptr(topk_weights), self.routed_scaling_factor, function, approximate, alpha, limit,
            up_offset, self._payload_code, _ptr(output), _ptr(self.workspace), self.workspace.numel(), _stream(),
        )
