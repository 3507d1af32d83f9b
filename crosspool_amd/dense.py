"""Dense FFN operator over caller-owned storage (eager launches of the native kernels).

Mirrors ``DenseExecutionPlan`` / ``Dense.run_into`` of
src/xpool/runtime/ffnagent/operators/dense.py:14-86 and the projection entry
of operators/linear.py:163-257.  Every launch goes to the HIP library on the
current torch stream; nothing here computes on the CPU.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from crosspool_amd import _native
from crosspool_amd.execution import DenseFfnExecutionSignature, WorkspaceLayout
from crosspool_amd.ffn import GateTransform, SiluActivation, activation_arguments
from crosspool_amd.weights import DenseFfnWeights


def _stream(stream: torch.cuda.Stream | None = None) -> ctypes.c_void_p:
    stream = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


_scratch: dict[tuple[int, int], torch.Tensor] = {}


def _projection_scratch(
    device: torch.device, stream: torch.cuda.Stream | None, rows: int, n: int, k: int, gated: bool
) -> tuple[ctypes.c_void_p | None, int]:
    """Scratch for the K-slice partial sums of a kernel-level projection.

    One buffer per (device, stream), grown on demand: calls ordered on one stream may reuse
    it (its contents do not matter on entry); calls on different streams may overlap, so
    they get separate buffers.
    """

    needed = _native.gemm_workspace_bytes(rows, n, k, gated)
    if needed == 0:
        return None, 0
    stream = stream if stream is not None else torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream)
    scratch = _scratch.get(key)
    if scratch is None or scratch.numel() < needed:
        scratch = torch.empty(needed, dtype=torch.uint8, device=device)
        _scratch[key] = scratch
    return ctypes.c_void_p(scratch.data_ptr()), scratch.numel()


def _require(tensor: torch.Tensor, name: str, dtype: torch.dtype, ndim: int) -> None:
    if tensor.device.type != "cuda":
        raise ValueError(f"{name} must be GPU-resident")
    if tensor.dtype is not dtype:
        raise ValueError(f"{name} must use {dtype}")
    if tensor.ndim != ndim:
        raise ValueError(f"{name} must have {ndim} dimensions")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def gate_up_silu(
    x: torch.Tensor,
    w_gate_up: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
    activation: SiluActivation = SiluActivation(),
    gate: GateTransform = GateTransform(),
    stream: torch.cuda.Stream | None = None,
) -> torch.Tensor:
    """``silu(bf16(x W_g^T)) * bf16(x W_u^T)`` rounded to bf16, W interleaved ``[2I, H]``."""

    _require(x, "x", torch.bfloat16, 2)
    _require(w_gate_up, "w_gate_up", torch.bfloat16, 2)
    rows, hidden = x.shape
    if w_gate_up.shape[1] != hidden or w_gate_up.shape[0] % 2:
        raise ValueError("w_gate_up must be [2I, H]")
    intermediate = w_gate_up.shape[0] // 2
    if out is None:
        out = torch.empty((rows, intermediate), dtype=torch.bfloat16, device=x.device)
    _require(out, "out", torch.bfloat16, 2)
    if tuple(out.shape) != (rows, intermediate):
        raise ValueError("out must be [rows, I]")
    alpha, limit, up_offset = activation_arguments(activation, gate)
    scratch, scratch_bytes = _projection_scratch(x.device, stream, rows, 2 * intermediate, hidden, True)
    _native.call(
        "xp_gemm_gate_up_silu",
        _ptr(x), rows, hidden, _ptr(w_gate_up), intermediate, _ptr(out), alpha, limit, up_offset, scratch,
        scratch_bytes, _stream(stream),
    )
    return out


def down(
    activated: torch.Tensor,
    w_down: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
    slots: torch.Tensor | None = None,
    stream: torch.cuda.Stream | None = None,
) -> torch.Tensor:
    """``bf16(h W_d^T)``; with ``slots`` row t is written to ``out[slots[t]]`` instead."""

    _require(activated, "activated", torch.bfloat16, 2)
    _require(w_down, "w_down", torch.bfloat16, 2)
    rows, intermediate = activated.shape
    hidden = w_down.shape[0]
    if w_down.shape[1] != intermediate:
        raise ValueError("w_down must be [H, I]")
    if out is None:
        if slots is not None:
            raise ValueError("a scattering down projection needs its destination")
        out = torch.empty((rows, hidden), dtype=torch.bfloat16, device=activated.device)
    _require(out, "out", torch.bfloat16, 2)
    if out.shape[1] != hidden or (slots is None and out.shape[0] != rows):
        raise ValueError("out must be [rows, H] (or [pool_rows, H] with slots)")
    if slots is not None:
        _require(slots, "slots", torch.int32, 1)
        if slots.numel() < rows:
            raise ValueError("slots must name one destination row per input row")
    scratch, scratch_bytes = _projection_scratch(activated.device, stream, rows, hidden, intermediate, False)
    _native.call(
        "xp_gemm_down",
        _ptr(activated), rows, intermediate, _ptr(w_down), hidden, _ptr(out), _ptr(slots), out.shape[0], scratch,
        scratch_bytes, _stream(stream),
    )
    return out


@dataclass(frozen=True, slots=True)
class DenseExecutionPlan:
    """Workspace of one Dense signature (operators/dense.py:14-52).

    Regions: the gathered (normalised) batch ``[capacity, H]`` and the
    activated intermediate ``[capacity, I]``; SiLU*mul is always fused into
    the gate_up epilogue, so no separate projected buffer exists.  Capacities
    whose projections split K across workgroups (sliced stream or split tile
    kernels) append the fp32 partial sums of the K ranges (``workspace_bytes``
    covers them, as GemmPlan's split-K workspace does in
    operators/linear.py:111-131).
    """

    signature: DenseFfnExecutionSignature
    workspace: WorkspaceLayout
    workspace_bytes: int

    @classmethod
    def prepare(cls, signature: DenseFfnExecutionSignature) -> DenseExecutionPlan:
        layout = signature.workspace_layout()
        native = _native.dense_workspace_bytes(
            signature.payload_row_capacity, signature.hidden_size, signature.local_intermediate_size
        )
        if native < layout.nbytes:
            raise RuntimeError(f"native workspace ({native} B) is smaller than the prepared layout ({layout.nbytes} B)")
        return cls(signature=signature, workspace=layout, workspace_bytes=native)


class Dense:
    """Eager Dense computation borrowing a prepared workspace (operators/dense.py:55-86)."""

    def __init__(self, plan: DenseExecutionPlan, workspace: torch.Tensor) -> None:
        if workspace.device.type != "cuda":
            raise ValueError("Dense workspace must reside on its execution device")
        if workspace.numel() < plan.workspace_bytes:
            raise ValueError("Dense workspace is smaller than the plan's workspace_bytes")
        self.plan = plan
        self.workspace = workspace
        self.batch, self.activated = plan.workspace.views(workspace)

    def run_into(self, *, hidden_states: torch.Tensor, layer_weights: DenseFfnWeights, output: torch.Tensor) -> None:
        """Write the complete rank-local partial of ``hidden_states`` into ``output``."""

        rows = hidden_states.shape[0]
        if rows > self.plan.signature.payload_row_capacity:
            raise ValueError("hidden states exceed the prepared row capacity")
        activated = self.activated[:rows]
        gate_up_silu(hidden_states, layer_weights.i_proj.values, out=activated)
        down(activated, layer_weights.o_proj.values, out=output)

    def step(
        self,
        *,
        pool: torch.Tensor,
        slots: torch.Tensor,
        layer_weights: DenseFfnWeights,
        norm_weight: torch.Tensor | None = None,
        eps: float = 1e-6,
        out_pool: torch.Tensor | None = None,
        fault_word: torch.Tensor | None = None,
    ) -> None:
        """Mailbox step: gather ``slots`` (+RMSNorm), Dense, scatter back into ``out_pool`` (default ``pool``)."""

        out_pool = pool if out_pool is None else out_pool
        _require(pool, "pool", torch.bfloat16, 2)
        _require(out_pool, "out_pool", torch.bfloat16, 2)
        _require(slots, "slots", torch.int32, 1)
        if out_pool.shape != pool.shape:
            raise ValueError("input and output mailboxes must have one shape")
        rows = slots.numel()
        if rows > self.plan.signature.payload_row_capacity:
            raise ValueError("slot count exceeds the prepared row capacity")
        if norm_weight is not None:
            _require(norm_weight, "norm_weight", torch.bfloat16, 1)
        if fault_word is not None:
            _require(fault_word, "fault_word", torch.int32, 1)
        signature = self.plan.signature
        _native.call(
            "xp_dense_step",
            _ptr(pool), _ptr(out_pool), pool.shape[0], _ptr(slots), rows, signature.hidden_size,
            signature.local_intermediate_size, _ptr(layer_weights.i_proj.values), _ptr(layer_weights.o_proj.values),
            _ptr(norm_weight), float(eps), _ptr(self.workspace), self.workspace.numel(), _ptr(fault_word), _stream(),
        )


def gather_rmsnorm(
    pool: torch.Tensor,
    slots: torch.Tensor,
    *,
    norm_weight: torch.Tensor | None = None,
    eps: float = 1e-6,
    out: torch.Tensor | None = None,
    fault_word: torch.Tensor | None = None,
    stream: torch.cuda.Stream | None = None,
) -> torch.Tensor:
    """Transport gather of mailbox rows, with the optional fused RMSNorm."""

    _require(pool, "pool", torch.bfloat16, 2)
    _require(slots, "slots", torch.int32, 1)
    rows = slots.numel()
    if out is None:
        out = torch.empty((rows, pool.shape[1]), dtype=torch.bfloat16, device=pool.device)
    _require(out, "out", torch.bfloat16, 2)
    if tuple(out.shape) != (rows, pool.shape[1]):
        raise ValueError("out must be [rows, H]")
    if norm_weight is not None:
        _require(norm_weight, "norm_weight", torch.bfloat16, 1)
        if norm_weight.numel() != pool.shape[1]:
            raise ValueError("norm weight must have one value per hidden column")
    _native.call(
        "xp_gather_rmsnorm",
        _ptr(pool), pool.shape[0], pool.shape[1], _ptr(slots), rows, _ptr(norm_weight), float(eps), _ptr(out),
        _ptr(fault_word), _stream(stream),
    )
    return out


def scatter(
    values: torch.Tensor,
    slots: torch.Tensor,
    pool: torch.Tensor,
    *,
    fault_word: torch.Tensor | None = None,
    stream: torch.cuda.Stream | None = None,
) -> torch.Tensor:
    """Transport scatter: ``pool[slots[i]] = values[i]``, bit-exact."""

    _require(values, "values", torch.bfloat16, 2)
    _require(slots, "slots", torch.int32, 1)
    _require(pool, "pool", torch.bfloat16, 2)
    if values.shape[1] != pool.shape[1] or slots.numel() != values.shape[0]:
        raise ValueError("values must be [len(slots), H] with the mailbox width")
    _native.call(
        "xp_scatter",
        _ptr(values), values.shape[0], values.shape[1], _ptr(slots), _ptr(pool), pool.shape[0], _ptr(fault_word),
        _stream(stream),
    )
    return pool


def copy_bytes(destination: torch.Tensor, source: torch.Tensor, *, stream: torch.cuda.Stream | None = None) -> None:
    """Byte copy of two equal-size device ranges (any alignment)."""

    if destination.nbytes != source.nbytes:
        raise ValueError("copy ranges differ in size")
    _native.call("xp_copy_bytes", _ptr(destination), _ptr(source), source.nbytes, _stream(stream))
