"""FfnAgent-owned Dense weight tensors (mirrors src/xpool/runtime/ffnagent/weights.py)."""

from __future__ import annotations

from dataclasses import dataclass

import torch


def validate_weight_tensor(tensor: torch.Tensor, *, name: str) -> None:
    """Device-resident, contiguous, positive-sized, 16-byte aligned (weights.py:232-247)."""

    if tensor.device.type != "cuda":
        raise ValueError(f"{name} must be GPU-resident")
    if not tensor.is_contiguous() or any(size <= 0 for size in tensor.shape):
        raise ValueError(f"{name} must have contiguous positive dimensions")
    if tensor.data_ptr() % 16:
        raise ValueError(f"{name} must be 16-byte aligned")


PAYLOAD_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


@dataclass(frozen=True, slots=True)
class ProjectionWeights:
    """One projection's retained storage (weights.py:294-328).

    ``values`` is ``[N, K]`` (bf16, fp16 or fp32) with K contiguous; ``bias`` is an optional
    fp32 ``[N]`` vector added to the fp32 sum before any rounding.  Scales (MXFP4) are not
    part of this build and are refused.  The FfnAgent's captured templates take bf16 values
    without a bias (``DenseFfnWeights.template_ready``); the operator path
    (``crosspool_amd.operators``) takes the rest.
    """

    values: torch.Tensor
    scales: torch.Tensor | None = None
    bias: torch.Tensor | None = None

    def __post_init__(self) -> None:
        if self.values.device.type != "cuda" or not self.values.is_contiguous() or self.values.ndim != 2:
            raise ValueError("projection values must be a contiguous GPU matrix")
        if any(size <= 0 for size in self.values.shape):
            raise ValueError("projection values must have positive dimensions")
        if self.values.dtype not in PAYLOAD_DTYPES:
            raise ValueError("projection values must be bf16, fp16 or fp32")
        if self.scales is not None:
            raise ValueError("quantised projections are not supported on the MI355X Dense path")
        if self.bias is not None:
            if self.bias.dtype is not torch.float32 or tuple(self.bias.shape) != (self.values.shape[0],):
                raise ValueError("a projection bias must be an fp32 vector with one value per output row")
            if self.bias.device != self.values.device or not self.bias.is_contiguous():
                raise ValueError("a projection bias must be contiguous on the values' device")


@dataclass(frozen=True, slots=True)
class DenseFfnWeights:
    """Retained input and output resources of one local Dense shard (weights.py:331-366).

    ``i_proj.values`` is ``[2 I, H]`` with INTERLEAVED Gate/Up rows (row 2j =
    gate_j, row 2j+1 = up_j, runtime/ffnagent/preparation.py:227);
    ``o_proj.values`` is ``[H, I]``.
    """

    i_proj: ProjectionWeights
    o_proj: ProjectionWeights

    def __post_init__(self) -> None:
        rows, hidden = self.i_proj.values.shape
        out_hidden, intermediate = self.o_proj.values.shape
        if rows not in (intermediate, 2 * intermediate) or out_hidden != hidden:
            raise ValueError("Dense projections disagree: i_proj must be [2I, H] (gated) or [I, H] and o_proj [H, I]")
        if self.o_proj.values.device != self.i_proj.values.device:
            raise ValueError("Dense projections must share one device")
        if self.i_proj.values.data_ptr() == self.o_proj.values.data_ptr():
            raise ValueError("Dense projections must own independent storages")

    @property
    def hidden_size(self) -> int:
        return int(self.i_proj.values.shape[1])

    @property
    def local_intermediate_size(self) -> int:
        return int(self.o_proj.values.shape[1])

    @property
    def device(self) -> torch.device:
        return self.i_proj.values.device

    @property
    def payload_dtype(self) -> torch.dtype:
        return self.i_proj.values.dtype

    @property
    def template_ready(self) -> bool:
        """Whether the FfnAgent's captured templates can run these weights: gated
        INTERLEAVED i_proj ``[2I, H]`` and o_proj of one payload dtype (bf16 or fp16,
        ffn.hpp:83-85), no biases, 16-byte aligned rows."""

        i_proj, o_proj = self.i_proj, self.o_proj
        return (
            i_proj.values.dtype in (torch.bfloat16, torch.float16) and o_proj.values.dtype is i_proj.values.dtype
            and i_proj.bias is None and o_proj.bias is None
            and i_proj.values.shape[0] == 2 * self.local_intermediate_size
            and self.hidden_size % 8 == 0 and self.local_intermediate_size % 8 == 0
            and i_proj.values.data_ptr() % 16 == 0 and o_proj.values.data_ptr() % 16 == 0
        )

    @classmethod
    def from_tensors(cls, gate_up: torch.Tensor, down: torch.Tensor) -> DenseFfnWeights:
        return cls(i_proj=ProjectionWeights(gate_up), o_proj=ProjectionWeights(down))


def interleave_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Prepare the INTERLEAVED i_proj from separate Gate and Up ``[I, H]`` matrices.

    The loader's Gate/Up normalisation (runtime/ffnagent/preparation.py:194-241,
    src/xpool/ffn.py:57-68): row 2j = gate_j, row 2j+1 = up_j.
    """

    if gate.shape != up.shape or gate.ndim != 2:
        raise ValueError("gate and up must be matrices of one shape")
    return torch.stack((gate, up), dim=1).flatten(0, 1).contiguous()
