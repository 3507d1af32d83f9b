"""FfnAgent operators over caller-owned storage: Activation, Gemm and Dense.

Mirrors the reference's operator layer (CrossPool checkout):

- ``Activation`` -- operators/activation.py:87-207 (``fused`` epilogue description,
  ``apply_into`` standalone activation);
- ``GemmPlan`` / ``Gemm`` -- operators/linear.py:28-257 (a prepared projection with its
  scratch, replayed with the current layer's values and bias);
- ``DenseExecutionPlan`` / ``Dense`` -- operators/dense.py:14-86 (i_proj, then the
  standalone activation when no epilogue could be fused -- CONCATENATED Gate/Up order --,
  then o_proj).

Every launch goes to the HIP library on the current torch stream and allocates nothing
(the plan's workspace holds all scratch), so a ``run_into`` can be captured into a graph.
Projections of bf16 payloads with aligned shapes, no bias and either no epilogue or the
gated SiLU epilogue over INTERLEAVED rows take the MFMA kernels (``xp_gemm_down`` /
``xp_gemm_gate_up_silu``); every other projection -- fp16 and fp32 payloads, odd K or N, a
bias, ReLU / GELU epilogues -- takes ``xp_projection``.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from crosspool_amd import _native
from crosspool_amd.execution import WorkspaceLayout
from crosspool_amd.ffn import GateTransform, GateUpOrder, GeluActivation, ReluActivation, SiluActivation
from crosspool_amd.weights import DenseFfnWeights, ProjectionWeights

ActivationSpec = SiluActivation | ReluActivation | GeluActivation

_DTYPE_CODES = {torch.bfloat16: _native.XP_DTYPE_BF16, torch.float16: _native.XP_DTYPE_F16,
                torch.float32: _native.XP_DTYPE_F32}
_ORDER_CODES = {GateUpOrder.CONCATENATED: _native.XP_GATE_UP_CONCATENATED,
                GateUpOrder.INTERLEAVED: _native.XP_GATE_UP_INTERLEAVED}


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


@dataclass(frozen=True, slots=True)
class TensorLayout:
    """Address-free shape, dtype and neutral fill value of one tensor (xpool.quantization.TensorLayout)."""

    shape: tuple[int, ...]
    dtype: torch.dtype
    zero_value: float = 0

    @property
    def nbytes(self) -> int:
        return math.prod(self.shape) * self.dtype.itemsize


@dataclass(frozen=True, slots=True)
class ProjectionLayout:
    """Unquantized projection: values ``[N, K]``, optional fp32 bias ``[N]`` and, for the
    i_proj of a gated layer, the physical Gate/Up row order (weights.py:52-92)."""

    values: TensorLayout
    bias: TensorLayout | None = None
    gate_up_order: GateUpOrder | None = None

    def zero_probe(self, device: torch.device) -> ProjectionWeights:
        """Shape-equivalent zero resources, as the Control Capture Probes (weights.py:66-87)."""

        values = torch.full(self.values.shape, self.values.zero_value, dtype=self.values.dtype, device=device)
        bias = None if self.bias is None else torch.full(self.bias.shape, self.bias.zero_value,
                                                         dtype=self.bias.dtype, device=device)
        return ProjectionWeights(values=values, bias=bias)

    @classmethod
    def of(cls, projection: ProjectionWeights, *, order: GateUpOrder | None = None) -> ProjectionLayout:
        bias = projection.bias
        return cls(
            values=TensorLayout(tuple(projection.values.shape), projection.values.dtype),
            bias=None if bias is None else TensorLayout(tuple(bias.shape), bias.dtype),
            gate_up_order=order,
        )


@dataclass(frozen=True, slots=True)
class Activation:
    """A layer's activation and optional Gate/Up combination (activation.py:87-96)."""

    function: ActivationSpec
    gate: GateTransform | None

    @property
    def supports_inplace(self) -> bool:
        """A standalone ungated activation may reuse its input (activation.py:94-97)."""

        return self.gate is None

    def descriptor(self) -> _native.ActivationDesc:
        function = self.function
        gate = self.gate
        desc = _native.ActivationDesc()
        desc.function = int(function.kind)
        desc.approximate_tanh = int(isinstance(function, GeluActivation) and function.approximate == "tanh")
        desc.alpha = float(function.alpha) if isinstance(function, SiluActivation) else 1.0
        desc.gated = int(gate is not None)
        desc.has_limit = int(gate is not None and gate.limit is not None)
        desc.limit = float(gate.limit) if gate is not None and gate.limit is not None else 0.0
        desc.up_offset = float(gate.up_offset) if gate is not None else 0.0
        return desc

    def fused(self, *, order: GateUpOrder | None) -> Activation | None:
        """The activation as a projection epilogue, or None when it cannot be one: a gated
        activation fuses only over adjacent (INTERLEAVED) Gate/Up rows (activation.py:112-131)."""

        if self.gate is not None and order is not GateUpOrder.INTERLEAVED:
            return None
        return self

    def apply_into(self, *, inputs: torch.Tensor, output: torch.Tensor, order: GateUpOrder | None) -> None:
        """Standalone activation into contiguous bf16 / fp16 storage (activation.py:175-207).

        Inputs already include the projection rounding.  Ungated input and output may be the
        same tensor; a gated input has twice the output width and needs separate storage.
        """

        if self.gate is not None and order is None:
            raise ValueError("gated activation requires a Gate/Up order")
        if inputs.dtype != output.dtype or inputs.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("activation payloads must share one bf16 or fp16 dtype")
        if not inputs.is_contiguous() or not output.is_contiguous():
            raise ValueError("activation payloads must be contiguous")
        width = output.shape[-1]
        rows = output.numel() // width if width else 0
        if inputs.numel() != output.numel() * (2 if self.gate is not None else 1):
            raise ValueError("gated inputs hold two values per output, ungated ones one")
        desc = self.descriptor()
        _native.call(
            "xp_activation", _ptr(inputs), _ptr(output), rows, width, _DTYPE_CODES[output.dtype],
            _ORDER_CODES.get(order, 0), ctypes.byref(desc), _stream(),
        )


@dataclass(frozen=True, slots=True)
class GemmPlan:
    """Address-free operand layout, epilogue and scratch of one projection (linear.py:28-131)."""

    input_layout: TensorLayout
    weight_layout: ProjectionLayout
    output_layout: TensorLayout
    fused_activation: Activation | None
    workspace: WorkspaceLayout
    kernel: str  # "gate_up_silu" or "down" (MFMA kernels) or "projection" (xp_projection)

    @classmethod
    def prepare(
        cls,
        *,
        input_layout: TensorLayout,
        weight_layout: ProjectionLayout,
        result_layout: TensorLayout,
        activation: Activation | None,
    ) -> GemmPlan:
        """Choose the kernel and size its scratch; the fused epilogue keeps the projection
        rounding to the result dtype (linear.py:42-96)."""

        if len(input_layout.shape) != 2 or len(result_layout.shape) != 2 or len(weight_layout.values.shape) != 2:
            raise ValueError("GEMM input, weights and result must be matrices")
        rows, hidden = input_layout.shape
        width, reduction = weight_layout.values.shape
        if reduction != hidden:
            raise ValueError("GEMM weights disagree with the input width")
        dtype = input_layout.dtype
        if weight_layout.values.dtype is not dtype or result_layout.dtype is not dtype:
            raise ValueError("GEMM input, weights and result must share one payload dtype")
        if activation is not None and activation.gate is not None and weight_layout.gate_up_order is None:
            raise ValueError("gated GEMM preparation requires physical Gate/Up order")
        fused = None if activation is None else activation.fused(order=weight_layout.gate_up_order)
        gated_epilogue = fused is not None and fused.gate is not None
        output_width = width // 2 if gated_epilogue else width
        if result_layout.shape != (rows, output_width):
            raise ValueError(f"GEMM result must be {(rows, output_width)}")
        # The MFMA kernels take bf16 rows of 16-byte multiples, no bias, and at most 16384 columns
        # on the side the C ABI treats as the hidden size (N for down, K for gate_up).
        aligned = dtype is torch.bfloat16 and weight_layout.bias is None and hidden % 8 == 0 and width % 16 == 0
        if aligned and fused is None and width <= 16384:
            kernel = "down"
            scratch = _native.gemm_workspace_bytes_upto(rows, width, hidden, False)
        elif aligned and gated_epilogue and isinstance(fused.function, SiluActivation) and hidden <= 16384:
            kernel = "gate_up_silu"
            scratch = _native.gemm_workspace_bytes_upto(rows, width, hidden, True)
        else:
            kernel = "projection"
            scratch = 0
        regions = ((torch.uint8, (scratch,)),) if scratch else ()
        return cls(
            input_layout=input_layout,
            weight_layout=weight_layout,
            output_layout=TensorLayout((rows, output_width), dtype),
            fused_activation=fused,
            workspace=WorkspaceLayout.from_regions(regions),
            kernel=kernel,
        )


class Gemm:
    """Capture-time projection borrowing its plan and scratch (linear.py:134-257)."""

    def __init__(self, plan: GemmPlan, workspace: torch.Tensor) -> None:
        if workspace.device.type != "cuda":
            raise ValueError("GEMM scratch must reside on its execution device")
        self.plan = plan
        views = plan.workspace.views(workspace) if plan.workspace.nbytes else ()
        self.scratch = views[0] if views else None

    def run_into(self, inputs: torch.Tensor, projection: ProjectionWeights, *, output: torch.Tensor) -> None:
        """Write the prepared projection of ``inputs`` with the current layer's values and bias."""

        plan = self.plan
        rows, hidden = plan.input_layout.shape
        if inputs.shape[0] > rows or inputs.shape[1] != hidden or inputs.dtype is not plan.input_layout.dtype:
            raise ValueError("GEMM input disagrees with the prepared layout")
        if tuple(projection.values.shape) != plan.weight_layout.values.shape:
            raise ValueError("GEMM weights disagree with the prepared layout")
        if (projection.bias is None) != (plan.weight_layout.bias is None):
            raise ValueError("GEMM bias presence disagrees with the prepared layout")
        live = inputs.shape[0]
        width = projection.values.shape[0]
        scratch = _ptr(self.scratch)
        scratch_bytes = 0 if self.scratch is None else self.scratch.numel()
        if plan.kernel == "down":
            _native.call(
                "xp_gemm_down", _ptr(inputs), live, hidden, _ptr(projection.values), width, _ptr(output), None, live,
                scratch, scratch_bytes, _stream(),
            )
        elif plan.kernel == "gate_up_silu":
            function, gate = plan.fused_activation.function, plan.fused_activation.gate
            _native.call(
                "xp_gemm_gate_up_silu", _ptr(inputs), live, hidden, _ptr(projection.values), width // 2,
                _ptr(output), float(function.alpha), float(gate.limit or 0.0), float(gate.up_offset), scratch,
                scratch_bytes, _stream(),
            )
        else:
            desc = None if plan.fused_activation is None else plan.fused_activation.descriptor()
            _native.call(
                "xp_projection", _ptr(inputs), live, hidden, _ptr(projection.values), width, _ptr(projection.bias),
                _ptr(output), _DTYPE_CODES[inputs.dtype], None if desc is None else ctypes.byref(desc), _stream(),
            )


@dataclass(frozen=True, slots=True)
class DenseSignature:
    """Dense operator identity (execution.py:73-95 DenseFfnExecutionSignature): payload
    dtype and capacity, widths, activation and the two projection layouts."""

    payload_dtype: torch.dtype
    payload_row_capacity: int
    hidden_size: int
    local_intermediate_size: int
    activation: Activation
    i_proj: ProjectionLayout
    o_proj: ProjectionLayout

    @property
    def payload_shape(self) -> tuple[int, int]:
        return self.payload_row_capacity, self.hidden_size


@dataclass(frozen=True, slots=True)
class DenseExecutionPlan:
    """Two prepared projections and their shared intermediate storage (dense.py:14-52)."""

    signature: DenseSignature
    i_proj: GemmPlan
    o_proj: GemmPlan
    workspace: WorkspaceLayout

    @classmethod
    def prepare(cls, signature: DenseSignature) -> DenseExecutionPlan:
        dtype = signature.payload_dtype
        capacity = signature.payload_row_capacity
        activated = TensorLayout((capacity, signature.local_intermediate_size), dtype)
        i_proj = GemmPlan.prepare(
            input_layout=TensorLayout(signature.payload_shape, dtype),
            weight_layout=signature.i_proj,
            result_layout=activated if signature.activation.fused(order=signature.i_proj.gate_up_order) is not None
            else TensorLayout((capacity, signature.i_proj.values.shape[0]), dtype),
            activation=signature.activation,
        )
        o_proj = GemmPlan.prepare(
            input_layout=activated, weight_layout=signature.o_proj,
            result_layout=TensorLayout(signature.payload_shape, dtype), activation=None,
        )
        regions = [(dtype, i_proj.output_layout.shape)]
        if i_proj.fused_activation is None and not signature.activation.supports_inplace:
            regions.append((dtype, activated.shape))
        regions += [(torch.uint8, (i_proj.workspace.nbytes,)), (torch.uint8, (o_proj.workspace.nbytes,))]
        return cls(signature, i_proj, o_proj, WorkspaceLayout.from_regions(tuple(regions)))


class Dense:
    """Capture-time Dense computation over a prepared workspace (dense.py:55-86)."""

    def __init__(self, plan: DenseExecutionPlan, workspace: torch.Tensor) -> None:
        views = plan.workspace.views(workspace)
        self.plan = plan
        self.projected = views[0]
        separate = plan.i_proj.fused_activation is None and not plan.signature.activation.supports_inplace
        self.activated = views[1] if separate else self.projected
        self.i_proj = Gemm(plan.i_proj, views[-2])
        self.o_proj = Gemm(plan.o_proj, views[-1])

    def run_into(self, *, hidden_states: torch.Tensor, layer_weights: DenseFfnWeights, output: torch.Tensor) -> None:
        """Write the complete rank-local partial of ``hidden_states`` into ``output``."""

        rows = hidden_states.shape[0]
        projected = self.projected[:rows]
        self.i_proj.run_into(hidden_states, layer_weights.i_proj, output=projected)
        activated = self.activated[:rows]
        if self.plan.i_proj.fused_activation is None:
            self.plan.signature.activation.apply_into(
                inputs=projected, output=activated, order=self.plan.i_proj.weight_layout.gate_up_order
            )
        self.o_proj.run_into(activated, layer_weights.o_proj, output=output)
