"""torch-CPU / numpy restatement of the reference FfnAgent Dense-FFN path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Every function cites the
reference file:line whose behaviour it restates (paths relative to the
CrossPool checkout).  Floating-point work follows the reference's own
qualification oracle: fp64 projections, payload-dtype (bf16) stage rounding,
fp32 SiLU*mul.  Index work (gather / scatter / copy) is plain numpy on the raw
16-bit patterns, so it is bit-exact by construction.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

NORMALIZED_RMSE_DENOMINATOR_FLOOR = 1e-12  # support/ffn.py:17
FFN_OUTPUT_NORMALIZED_RMSE_LIMIT = 0.01  # support/ffn.py:23
FFN_OUTPUT_MAXIMUM_SCALED_ERROR_LIMIT = 0.10  # support/ffn.py:24
OPERATOR_ALIGNMENT_BYTES = 16  # runtime/ffnagent/execution.py:16


# --------------------------------------------------------------------------- #
# bit helpers
# --------------------------------------------------------------------------- #
def bf16_bits(tensor: torch.Tensor) -> np.ndarray:
    """Raw uint16 patterns of a bf16 CPU tensor (no rounding)."""

    return tensor.contiguous().view(torch.int16).numpy().view(np.uint16)


def bf16_from_bits(bits: np.ndarray, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Inverse of :func:`bf16_bits`; ``dtype`` names the 16-bit payload (bf16 or fp16)."""

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(dtype)


def bf16_ulp(values: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at |values| (8 significant bits)."""

    magnitude = values.abs().float().clamp_min(2.0**-126)
    exponent = torch.floor(torch.log2(magnitude))
    return torch.pow(2.0, exponent - 7)


def f16_ulp(values: torch.Tensor) -> torch.Tensor:
    """Spacing of fp16 values at |values| (11 significant bits; 2^-24 below 2^-14)."""

    magnitude = values.abs().float().clamp_min(2.0**-14)
    exponent = torch.floor(torch.log2(magnitude))
    return torch.pow(2.0, exponent - 10)


# --------------------------------------------------------------------------- #
# Transport: byte copy, gather, scatter
# --------------------------------------------------------------------------- #
def copy_bytes(destination: np.ndarray, source: np.ndarray) -> None:
    """Byte copy of equal-size ranges.

    Restates ``xpool::utils::cooperative::copy`` (src/cext-include/xpool/utils/
    cooperative.cuh:37-55): sizes must match, an empty range is a no-op, the
    aligned / unaligned branches are the same bytes.
    """

    if destination.nbytes != source.nbytes:
        raise ValueError("copy ranges differ in size")  # cooperative.cuh:40 abort_if
    destination.view(np.uint8)[...] = source.view(np.uint8)


def gather(pool: torch.Tensor, slots: np.ndarray) -> torch.Tensor:
    """``out[i, :] = pool[slots[i], :]`` on raw bit patterns.

    Generalises the reference's contiguous row-prefix staging copy
    (src/cext/transport/instance.cu:83-84, src/cext/fabric/atnagent.cu:215):
    identity slots ``0..T-1`` reproduce it exactly.
    """

    bits = bf16_bits(pool)
    slots = np.asarray(slots, dtype=np.int64)
    if slots.size and (slots.min() < 0 or slots.max() >= bits.shape[0]):
        raise IndexError("slot id outside the mailbox pool")
    return bf16_from_bits(bits[slots].copy(), pool.dtype)


def scatter(pool: torch.Tensor, slots: np.ndarray, rows: torch.Tensor) -> torch.Tensor:
    """Return a copy of ``pool`` with ``pool[slots[i], :] = rows[i, :]``.

    Restates the output copy back into the caller's rows
    (src/cext/fabric/atnagent.cu:275, src/cext/transport/instance.cu:184-186),
    generalised from a prefix to slot ids.  Slot ids must be distinct.
    """

    if rows.dtype is not pool.dtype:
        raise ValueError("scatter rows must have the mailbox payload dtype")
    bits = bf16_bits(pool).copy()
    slots = np.asarray(slots, dtype=np.int64)
    if len(set(slots.tolist())) != slots.size:
        raise ValueError("scatter slot ids must be distinct")
    bits[slots] = bf16_bits(rows)
    return bf16_from_bits(bits, pool.dtype)


# --------------------------------------------------------------------------- #
# RMSNorm (new fusion; textbook formula)
# --------------------------------------------------------------------------- #
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``payload(x * rsqrt(mean(x^2) + eps) * w)`` with fp32 math, in x's payload dtype (bf16
    or fp16).

    The reference path has no RMSNorm (SGLang applies ``post_attention_layernorm``
    before the shim: src/xpool/integrations/sglang/models/qwen2.py:125-126).
    This is the textbook formula as SGLang's native RMSNorm evaluates it: fp32
    mean of squares, ``1/sqrt(. + eps)``, multiply by x then by the weight in
    fp32, one rounding to the payload dtype.  Parity with SGLang's kernel is unpinned.
    """

    xf = x.float()
    variance = xf.pow(2).mean(dim=-1, keepdim=True)
    inverse = 1.0 / torch.sqrt(variance + eps)
    return ((xf * inverse) * weight.float()).to(x.dtype)


# --------------------------------------------------------------------------- #
# Gated SiLU and the Dense partial
# --------------------------------------------------------------------------- #
def silu(value: torch.Tensor, alpha: float = 1.0) -> torch.Tensor:
    """``v / (1 + exp(-alpha v))`` in fp32 (operators/activation.py:31-34)."""

    value = value.float()
    return value / (1 + torch.exp(-alpha * value))


def gated_silu(
    gate: torch.Tensor,
    up: torch.Tensor,
    *,
    alpha: float = 1.0,
    limit: float | None = None,
    up_offset: float = 0.0,
    dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """Gated activation in fp32, rounded to the payload ``dtype`` (bf16 or fp16).

    operators/activation.py:37-51 (``compute_gated``): Gate clipped above at
    ``limit``, Up clamped to ``[-limit, limit]``, ``silu(gate) * (up + up_offset)``;
    the result is stored into the payload-dtype activated buffer
    (operators/dense.py:27-29).  Defaults are the Dense path's
    ``GateTransform()`` (src/xpool/ffn.py:130-137).
    """

    gate = gate.float()
    up = up.float()
    if limit is not None:
        gate = torch.clamp(gate, max=limit)
        up = torch.clamp(up, -limit, limit)
    return (silu(gate, alpha) * (up + up_offset)).to(dtype)


def activation_function(value: torch.Tensor, function: str, *, alpha: float = 1.0,
                        approximate: str = "none") -> torch.Tensor:
    """One activation in fp32 (operators/activation.py:19-41).

    ``relu``: the value where it is > 0 or NaN (payload kept), +0 otherwise
    (``compute_relu``, activation.py:19-27); ``silu``: ``v / (1 + exp(-alpha v))``
    (``compute_silu``); ``gelu``: ``0.5 v (1 + erf(v / sqrt 2))`` or, approximated,
    ``0.5 v (1 + tanh(0.7978845608028654 (v + 0.044715 v^3)))`` (``compute_gelu``).
    """

    value = value.float()
    if function == "relu":
        return torch.where((value > 0) | (value != value), value, torch.zeros_like(value))
    if function == "silu":
        return value / (1 + torch.exp(-alpha * value))
    if function == "gelu":
        if approximate == "tanh":
            inner = 0.7978845608028654 * (value + 0.044715 * value * value * value)
            return 0.5 * value * (1 + torch.tanh(inner))
        return 0.5 * value * (1 + torch.erf(value * 0.7071067811865476))
    raise ValueError(f"unknown activation {function!r}")


def relu_bits(values: torch.Tensor) -> torch.Tensor:
    """Ungated ReLU of bf16 / fp16 values on their raw patterns (activation.py:19-27, 80-82):
    the pattern where the value is > 0 or NaN, +0 otherwise."""

    bits = values.contiguous().view(torch.int16)
    keep = (values.float() > 0) | (values.float() != values.float())
    return torch.where(keep, bits, torch.zeros_like(bits)).view(values.dtype)


def standalone_activation(inputs: torch.Tensor, *, width: int, function: str, gated: bool, order: str | None = None,
                          alpha: float = 1.0, approximate: str = "none", limit: float | None = None,
                          up_offset: float = 0.0) -> torch.Tensor:
    """``activation_kernel`` (operators/activation.py:55-84) over projected bf16 / fp16 values.

    Gated: Gate and Up of output column j are inputs ``[2j, 2j + 1]`` (INTERLEAVED) or
    ``[j, width + j]`` (CONCATENATED) of the row, combined by ``compute_gated``
    (activation.py:44-51); the fp32 result is stored in the payload dtype.  Ungated ReLU is
    the bitwise rule of :func:`relu_bits`; other ungated functions compute in fp32.
    """

    dtype = inputs.dtype
    rows = inputs.numel() // (2 * width if gated else width)
    if not gated:
        flat = inputs.reshape(rows, width)
        if function == "relu":
            return relu_bits(flat)
        return activation_function(flat, function, alpha=alpha, approximate=approximate).to(dtype)
    pairs = inputs.reshape(rows, 2 * width)
    if order == "interleaved":
        gate, up = pairs[:, 0::2], pairs[:, 1::2]
    elif order == "concatenated":
        gate, up = pairs[:, :width], pairs[:, width:]
    else:
        raise ValueError("gated activation requires a Gate/Up order")
    return gated_activation(gate, up, function=function, alpha=alpha, approximate=approximate, limit=limit,
                            up_offset=up_offset).to(dtype)


def gated_activation(gate: torch.Tensor, up: torch.Tensor, *, function: str, alpha: float = 1.0,
                     approximate: str = "none", limit: float | None = None, up_offset: float = 0.0) -> torch.Tensor:
    """``compute_gated`` (activation.py:44-51) in fp32: Gate clipped above at ``limit``, Up to
    ``[-limit, limit]``, ``f(gate) * (up + up_offset)``; fp32 result."""

    gate = gate.float()
    up = up.float()
    if limit is not None:
        gate = torch.clamp(gate, max=limit)
        up = torch.clamp(up, -limit, limit)
    return activation_function(gate, function, alpha=alpha, approximate=approximate) * (up + up_offset)


def projection_reference(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None, *,
                         function: str | None = None, gated: bool = False, **activation) -> torch.Tensor:
    """A projection with the reference's epilogue (operators/linear.py:42-96, simt.py:13-45,
    activation.py:112-173), the sum in fp64.

    ``value = x . w^T + bias``; without an activation the value is rounded once to the payload
    dtype; with one it is rounded to the payload dtype (the projection rounding point), then
    activated in fp32 (gated: INTERLEAVED Gate/Up pairs), then rounded to the payload dtype.
    """

    dtype = x.dtype
    value = x.double() @ w.double().t()
    if bias is not None:
        value = value + bias.double()
    if function is None:
        return value.to(dtype)
    rounded = value.to(dtype)
    if gated:
        return gated_activation(rounded[:, 0::2], rounded[:, 1::2], function=function, **activation).to(dtype)
    return activation_function(rounded, function, **{k: v for k, v in activation.items()
                                                     if k in ("alpha", "approximate")}).to(dtype)


def dense_partial_reference(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor) -> torch.Tensor:
    """Dense partial with fp64 projections and payload stage rounding.

    src/xpool-dev/xtest/harness/native/ffn/qualification.py:290-314
    (``dense_partial_reference``): fp64 gate and up projections rounded to the
    payload dtype, ``silu(g.float()) * u.float()`` rounded to the payload
    dtype, fp64 down projection rounded to the payload dtype.  ``w_gate_up``
    is the prepared INTERLEAVED i_proj (row 2j = gate_j, row 2j+1 = up_j;
    runtime/ffnagent/preparation.py:227, qualification.py:259) and ``w_down``
    the o_proj ``[H, I]``.  The fp64 -> bf16 conversion is torch's (through
    fp32), as in the reference.
    """

    x64 = x.double()
    projected = torch.mm(x64, w_gate_up.double().t())
    gate = projected[:, 0::2].to(x.dtype)
    up = projected[:, 1::2].to(x.dtype)
    activated = gated_silu(gate, up, dtype=x.dtype)
    return torch.mm(activated.double(), w_down.double().t()).to(x.dtype)


def dense_fp32(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor) -> torch.Tensor:
    """Pure fp32 Dense FFN with no intermediate rounding; fp32 result.

    The north star's "fp32 reference": same formula as
    :func:`dense_partial_reference` without any payload-dtype stage.
    """

    projected = torch.mm(x.float(), w_gate_up.float().t())
    activated = silu(projected[:, 0::2]) * projected[:, 1::2]
    return torch.mm(activated, w_down.float().t())


def dense_stage_fp32(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor) -> torch.Tensor:
    """fp32-accumulated Dense with the reference's stage rounding (bf16 result).

    The CPU-baseline restatement: the formula of
    src/xpool-dev/xtest/harness/native/ffn/qualification.py:290-314 and
    tests/suites/integration/runtime/ffnagent/test_operators.py:66-69 with
    fp32 math on bf16-stored tensors (multi-threaded torch CPU matmuls).
    """

    projected = torch.mm(x.float(), w_gate_up.float().t())
    gate = projected[:, 0::2].to(torch.bfloat16)
    up = projected[:, 1::2].to(torch.bfloat16)
    activated = gated_silu(gate, up)
    return torch.mm(activated.float(), w_down.float().t()).to(torch.bfloat16)


def mailbox_step(
    pool: torch.Tensor,
    slots: np.ndarray,
    w_gate_up: torch.Tensor,
    w_down: torch.Tensor,
    *,
    norm_weight: torch.Tensor | None,
    eps: float = 1e-6,
    dense=dense_partial_reference,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One FfnAgent step over a mailbox: gather (+RMSNorm) -> Dense -> scatter.

    Returns ``(new_pool, normalized_rows, ffn_rows)``.  The Dense body is
    operators/dense.py:70-86; the copies are the Transport row copies named in
    :func:`gather` / :func:`scatter`.
    """

    rows = gather(pool, slots)
    if norm_weight is not None:
        rows = rmsnorm(rows, norm_weight, eps)
    out = dense(rows, w_gate_up, w_down)
    return scatter(pool, slots, out), rows, out


# --------------------------------------------------------------------------- #
# Deterministic weights (reference qualification builders)
# --------------------------------------------------------------------------- #
def dense_full_weights(
    *, hidden_size: int, intermediate_size: int, layer_ordinal: int = 0, dtype=torch.bfloat16
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``((arange + offset) mod 29 - 14) / 64`` gate, up and down tensors.

    qualification.py:317-336; every value is a multiple of 1/64 in [-14/64, 14/64],
    exactly representable in bf16.
    """

    def values(shape: tuple[int, int], offset: int) -> torch.Tensor:
        data = torch.arange(shape[0] * shape[1], dtype=torch.float32)
        return (((data + offset).remainder(29) - 14) / 64).reshape(shape).to(dtype)

    return (
        values((intermediate_size, hidden_size), 3 + layer_ordinal * 5),
        values((intermediate_size, hidden_size), 11 + layer_ordinal * 7),
        values((hidden_size, intermediate_size), 19 + layer_ordinal * 11),
    )


def interleave_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Row 2j = gate_j, row 2j+1 = up_j (qualification.py:259, ffn.py:57-68)."""

    return torch.stack((gate, up), dim=1).flatten(0, 1).contiguous()


def dense_layer_weights(
    *, hidden_size: int, intermediate_size: int, tp_size: int = 1, tp_rank: int = 0, layer_ordinal: int = 0
) -> tuple[torch.Tensor, torch.Tensor]:
    """One true-TP Dense shard: interleaved i_proj and column-sliced o_proj.

    qualification.py:235-264 (``dense_layer_weights``).
    """

    gate, up, down = dense_full_weights(
        hidden_size=hidden_size, intermediate_size=intermediate_size, layer_ordinal=layer_ordinal
    )
    width = intermediate_size // tp_size
    begin, end = tp_rank * width, (tp_rank + 1) * width
    return interleave_gate_up(gate[begin:end], up[begin:end]), down[:, begin:end].contiguous()


def ordered_partial_sum(partials: list[torch.Tensor]) -> torch.Tensor:
    """Fixed PE-order fold of bf16 TP partials (delivery.cu:74-83, ``ordered_sum``).

    Per element: an fp32 sum starting from +0, each partial widened to fp32 and added in
    list order with fp32 rounding after every add, then one cast to bf16 (nearest even).
    """

    total = np.zeros(partials[0].shape, dtype=np.float32)
    for partial in partials:
        total = (total + partial.float().numpy()).astype(np.float32)
    return torch.from_numpy(total).to(torch.bfloat16)


def dense_reference_sum(x: torch.Tensor, shards: list[tuple[torch.Tensor, torch.Tensor]]) -> torch.Tensor:
    """Ordered fp32 sum of TP partials, rounded once (qualification.py:267-287)."""

    result = torch.zeros_like(x, dtype=torch.float32)
    for w_gate_up, w_down in shards:
        result.add_(dense_partial_reference(x, w_gate_up, w_down))
    return result.to(x.dtype)


# --------------------------------------------------------------------------- #
# Seeded synthetic inputs
# --------------------------------------------------------------------------- #
def generate_hidden_states(rows: int, hidden_size: int, seed: int) -> torch.Tensor:
    """CPU ``torch.Generator(seed)`` normal sample cast to bf16 (support/ffn.py:42-61)."""

    generator = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn((rows, hidden_size), generator=generator).to(torch.bfloat16).contiguous()


def generate_layer(hidden_size: int, intermediate_size: int, seed: int, std: float = 0.02):
    """Interleaved ``W_gu [2I, H]`` and ``W_d [H, I]`` ~ N(0, std) bf16, norm weight 1+N(0, 0.1)."""

    generator = torch.Generator(device="cpu").manual_seed(seed)
    w_gate_up = (torch.randn((2 * intermediate_size, hidden_size), generator=generator) * std).to(torch.bfloat16)
    w_down = (torch.randn((hidden_size, intermediate_size), generator=generator) * std).to(torch.bfloat16)
    norm_weight = (1 + 0.1 * torch.randn((hidden_size,), generator=generator)).to(torch.bfloat16)
    return w_gate_up.contiguous(), w_down.contiguous(), norm_weight.contiguous()


def generate_slots(pool_rows: int, rows: int, seed: int) -> np.ndarray:
    """``randperm(pool_rows)[:rows]`` from a seeded CPU generator, as int32."""

    generator = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randperm(pool_rows, generator=generator)[:rows].to(torch.int32).numpy()


# --------------------------------------------------------------------------- #
# Capacity buckets and workspace geometry
# --------------------------------------------------------------------------- #
def derive_payload_row_capacities(maximum_row_capacity: int) -> tuple[int, ...]:
    """Powers of two below the maximum, then the exact maximum.

    runtime/ffnagent/execution.py:166-177.
    """

    if maximum_row_capacity <= 0:
        raise ValueError("maximum payload row capacity must be positive")
    capacities = []
    capacity = 1
    while capacity < maximum_row_capacity:
        capacities.append(capacity)
        capacity *= 2
    capacities.append(maximum_row_capacity)
    return tuple(capacities)


def select_capacity(capacities: tuple[int, ...], rows: int) -> int | None:
    """Smallest installed capacity containing ``rows`` (src/cext/ffnagent/runtime.cu:246-253)."""

    for capacity in capacities:
        if rows <= capacity:
            return capacity
    return None


def workspace_offsets(region_bytes: list[int]) -> tuple[tuple[int, ...], int]:
    """16-byte aligned region offsets and total (execution.py:46-58)."""

    offsets = []
    cursor = 0
    for size in region_bytes:
        if size:
            cursor = (cursor + OPERATOR_ALIGNMENT_BYTES - 1) // OPERATOR_ALIGNMENT_BYTES * OPERATOR_ALIGNMENT_BYTES
        offsets.append(cursor)
        cursor += size
    return tuple(offsets), cursor


# --------------------------------------------------------------------------- #
# Metrics
# --------------------------------------------------------------------------- #
@dataclass(frozen=True)
class Comparison:
    max_abs: float
    rel_l2: float
    normalized_rmse: float
    maximum_scaled_error: float
    over_abs: int
    over_ulp: int
    elements: int


def compare(reference: torch.Tensor, actual: torch.Tensor, *, abs_limit: float = 2e-2) -> Comparison:
    """Error metrics of ``actual`` against ``reference`` (both promoted to fp32).

    ``normalized_rmse`` and ``maximum_scaled_error`` restate
    src/xpool-dev/xtest/harness/support/ffn.py:344-357.  ``over_abs`` counts
    elements above ``abs_limit``; ``over_ulp`` counts elements that are off by
    more than ``max(abs_limit, one bf16 ulp of the reference)``.
    """

    ref = reference.float()
    act = actual.float()
    error = (act - ref).abs()
    scale = ref.square().mean().sqrt().clamp_min(NORMALIZED_RMSE_DENOMINATOR_FLOOR)
    nrmse = float(((act - ref).square().mean().sqrt() / scale).item())
    max_scaled = float((error / torch.maximum(ref.abs(), scale)).max().item()) if ref.numel() else 0.0
    rel_l2 = float(((act - ref).norm() / ref.norm().clamp_min(NORMALIZED_RMSE_DENOMINATOR_FLOOR)).item())
    bound = torch.maximum(torch.full_like(ref, abs_limit), bf16_ulp(ref))
    return Comparison(
        max_abs=float(error.max().item()) if ref.numel() else 0.0,
        rel_l2=rel_l2,
        normalized_rmse=nrmse,
        maximum_scaled_error=max_scaled,
        over_abs=int((error > abs_limit).sum().item()),
        over_ulp=int((error > bound).sum().item()),
        elements=ref.numel(),
    )


# --------------------------------------------------------------------------- #
# Roofline accounting
# --------------------------------------------------------------------------- #
def layer_flops(rows: int, hidden: int, intermediate: int) -> int:
    """GEMM flops of one Dense layer: ``6 T H I``."""

    return 6 * rows * hidden * intermediate


def layer_bytes(rows: int, hidden: int, intermediate: int) -> int:
    """Compulsory HBM bytes of one mailbox step (weights, norm, rows in/out, slot ids)."""

    return 6 * hidden * intermediate + 2 * hidden + 4 * rows * hidden + 4 * rows


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)

