"""Parity helpers shared by the GPU tests (tolerances stated here, used everywhere).

FFN output gates
----------------
* North star: rel-L2 <= 5e-3 against the pure-fp32 oracle (no intermediate
  rounding), and max-abs <= 2e-2 against the oracle with the reference's
  precision contract (qualification.py:290-314: fp64 projections, bf16 stage
  rounding of gate/up, activated h and the output).  Both sides round the
  output to bf16, so an element whose exact value sits next to a rounding
  boundary may come out one bf16 ulp apart; where one ulp exceeds 2e-2
  (|y| >= 4) such an element is allowed exactly one ulp, and at most 0.1 % of
  elements may exceed 2e-2 at all.  Without this allowance no bf16-output
  implementation can meet 2e-2 at Qwen3-8B scale (|y| reaches ~11, where half
  an ulp is already 0.031).
* Reference gates: ``assert_close(rtol=0.02, atol=0.1)``
  (tests/suites/integration/runtime/ffnagent/test_operators.py:70) and
  nRMSE <= 0.01, max-scaled error <= 0.10
  (src/xpool-dev/xtest/harness/support/ffn.py:23-26,357).
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import ffn_oracle as o

NORTH_STAR_MAX_ABS = 2e-2
NORTH_STAR_REL_L2 = 5e-3
MAX_FRACTION_OVER_ABS = 1e-3


def assert_bitwise_equal(actual: torch.Tensor, expected: torch.Tensor) -> None:
    a = actual.detach().cpu().contiguous().view(torch.int16)
    e = expected.detach().cpu().contiguous().view(torch.int16)
    assert a.shape == e.shape
    mismatches = int((a != e).sum().item())
    assert mismatches == 0, f"{mismatches} of {a.numel()} 16-bit patterns differ"


def assert_ffn_parity(actual: torch.Tensor, stage_reference: torch.Tensor, fp32_reference: torch.Tensor) -> None:
    actual = actual.detach().cpu()
    assert torch.isfinite(actual.float()).all(), "FFN output holds non-finite values"
    stage = o.compare(stage_reference, actual, abs_limit=NORTH_STAR_MAX_ABS)
    pure = o.compare(fp32_reference, actual.float(), abs_limit=NORTH_STAR_MAX_ABS)
    assert pure.rel_l2 <= NORTH_STAR_REL_L2, f"rel-L2 vs fp32 oracle {pure.rel_l2:.3e}"
    assert stage.over_ulp == 0, f"{stage.over_ulp} elements beyond max(2e-2, 1 ulp) (max-abs {stage.max_abs:.3e})"
    assert stage.over_abs <= MAX_FRACTION_OVER_ABS * stage.elements, f"{stage.over_abs} elements above 2e-2"
    assert stage.normalized_rmse <= o.FFN_OUTPUT_NORMALIZED_RMSE_LIMIT
    assert stage.maximum_scaled_error <= o.FFN_OUTPUT_MAXIMUM_SCALED_ERROR_LIMIT
    torch.testing.assert_close(actual, stage_reference, rtol=0.02, atol=0.1)


def assert_moe_parity(actual: torch.Tensor, stage_reference: torch.Tensor, fp32_reference: torch.Tensor,
                      slack: torch.Tensor) -> None:
    """The MoE Experts end-to-end bar.

    Every route output is rounded to the payload dtype before the row sum
    (test_operators.py:278), so an element may differ from the oracle by one ulp per route
    (scaled) plus one for the
    final rounding: ``slack`` is that bound per element (moe_oracle.rounding_slack).  A
    legitimate one-ulp flip of an activation (fp32 accumulation order, the epilogue's exp)
    moves every column of its route a little further, so up to 0.1 % of elements may exceed
    the slack; the stages themselves are checked rigorously by assert_moe_stages.  On top:
    rel-L2 <= 5e-3 against the pure-fp32 oracle (north star), the reference harness's
    nRMSE / max-scaled gates and its operator tolerance (rtol 0.02, atol 0.1).
    """

    actual = actual.detach().cpu()
    assert torch.isfinite(actual.float()).all(), "Experts output holds non-finite values"
    pure = o.compare(fp32_reference, actual.float())
    assert pure.rel_l2 <= NORTH_STAR_REL_L2, f"rel-L2 vs fp32 oracle {pure.rel_l2:.3e}"
    gap = (actual.float() - stage_reference.float()).abs()
    over = int((gap > slack).sum().item())
    assert over <= MAX_FRACTION_OVER_ABS * gap.numel(), (
        f"{over} elements beyond their rounding-point slack (max gap {gap.max().item():.3e})"
    )
    stage = o.compare(stage_reference, actual)
    assert stage.normalized_rmse <= o.FFN_OUTPUT_NORMALIZED_RMSE_LIMIT
    assert stage.maximum_scaled_error <= o.FFN_OUTPUT_MAXIMUM_SCALED_ERROR_LIMIT
    torch.testing.assert_close(actual, stage_reference, rtol=0.02, atol=0.1)


def assert_within_ulps(actual: torch.Tensor, expected: torch.Tensor, ulps: float = 1.0, exact_fraction: float = 0.99):
    """Elementwise |a - e| <= ulps * ulp(e) (ulp of e's dtype, bf16 or fp16) and at least
    ``exact_fraction`` bit-identical."""

    a = actual.detach().cpu().float()
    e = expected.detach().cpu().float()
    assert torch.isfinite(a).all()
    bound = ulps * _ulp(e, expected.dtype)
    over = int(((a - e).abs() > bound).sum().item())
    assert over == 0, f"{over} elements beyond {ulps} ulp (max diff {(a - e).abs().max().item():.3e})"
    exact = float((actual.detach().cpu().view(torch.int16) == expected.detach().cpu().view(torch.int16)).float().mean())
    assert exact >= exact_fraction, f"only {exact:.4f} of elements are bit-identical"


# --------------------------------------------------------------------------- #
# Rigorous bounds for the projections
#
# The kernels accumulate in fp32 and the oracle in fp64.  For a dot product S
# with magnitude sum M = sum |x_k w_k|, the fp32 result lies within
# delta = 2^-17 M of S (a bound of 128 full-magnitude fp32 roundings, far above
# the real blocked-summation error).  So a rounded projection must be one of
# the bf16 values in [floor_bf16(S - delta), ceil_bf16(S + delta)], and the
# gated activation must lie between the smallest and largest
# bf16(silu(g') * u') over the bf16 values g', u' reachable that way, widened
# by one bf16 ulp for the fp32 exp / divide of the epilogue.
# --------------------------------------------------------------------------- #
ACCUMULATION_BOUND = 2.0**-17


def _ulp(values: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return o.bf16_ulp(values) if dtype is torch.bfloat16 else o.f16_ulp(values)


def _key(b: torch.Tensor) -> torch.Tensor:
    """Order-preserving integer key of 16-bit floats (sign-magnitude bits: bf16 and fp16)."""

    bits = b.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    magnitude = bits & 0x7FFF
    return torch.where(bits >= 0x8000, -magnitude, magnitude)


def _from_key(key: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    bits = torch.where(key >= 0, key, 0x8000 | (-key))
    signed = bits - 0x10000 * (bits >= 0x8000).to(torch.int32)  # two's-complement int16 range
    return signed.to(torch.int16).view(dtype)


def step16(b: torch.Tensor, steps: int) -> torch.Tensor:
    """The value of b's dtype ``steps`` representable values above (negative: below) ``b``."""

    return _from_key(_key(b) + steps, b.dtype)


def floor16(v: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    b = v.to(dtype)
    return torch.where(b.double() > v, step16(b, -1), b)


def ceil16(v: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    b = v.to(dtype)
    return torch.where(b.double() < v, step16(b, 1), b)


def bf16_step(b: torch.Tensor, steps: int) -> torch.Tensor:
    return step16(b, steps)


def bf16_floor(v: torch.Tensor) -> torch.Tensor:
    return floor16(v, torch.bfloat16)


def bf16_ceil(v: torch.Tensor) -> torch.Tensor:
    return ceil16(v, torch.bfloat16)


def projection_interval(x: torch.Tensor, w: torch.Tensor, dtype: torch.dtype = torch.bfloat16,
                        bias: torch.Tensor | None = None):
    """Interval (of ``dtype``) a correctly implemented fp32-accumulated ``round(x w^T + bias)``
    must land in (the fp32 bias added to the fp32 sum: one more fp32 rounding)."""

    exact = x.double() @ w.double().t()
    delta = (x.double().abs() @ w.double().abs().t()) * ACCUMULATION_BOUND
    if bias is not None:
        exact = exact + bias.double()
        delta = delta + (exact.abs() + delta) * 2.0**-23
    return floor16(exact - delta, dtype), ceil16(exact + delta, dtype)


def _gated(gate: torch.Tensor, up: torch.Tensor, dtype: torch.dtype, *, function: str = "silu",
           approximate: str = "none", alpha: float = 1.0, limit: float | None = None,
           up_offset: float = 0.0) -> torch.Tensor:
    """The gated activation at the reference's rounding point: o.gated_silu for SiLU (the
    Dense oracle's), o.gated_activation rounded to ``dtype`` for ReLU and GELU."""

    if function == "silu":
        return o.gated_silu(gate, up, dtype=dtype, alpha=alpha, limit=limit, up_offset=up_offset)
    return o.gated_activation(gate, up, function=function, approximate=approximate, limit=limit,
                              up_offset=up_offset).to(dtype)


def assert_projection_within_bounds(actual: torch.Tensor, x: torch.Tensor, w: torch.Tensor, exact_fraction=0.99):
    a = actual.detach().cpu()
    lo, hi = projection_interval(x, w, a.dtype)
    assert torch.isfinite(a.float()).all()
    outside = int(((a.double() < lo.double()) | (a.double() > hi.double())).sum().item())
    assert outside == 0, f"{outside} of {a.numel()} projections outside their fp32-accumulation interval"
    nominal = (x.double() @ w.double().t()).to(a.dtype)
    exact = float((a.view(torch.int16) == nominal.view(torch.int16)).float().mean())
    assert exact >= exact_fraction, f"only {exact:.4f} of projections are bit-identical to the fp64 oracle"


def _candidates(lo: torch.Tensor, hi: torch.Tensor) -> list[torch.Tensor]:
    values = [lo, hi]
    for steps in (1, 2):
        stepped = step16(lo, steps)
        values.append(torch.where(stepped.double() <= hi.double(), stepped, hi))
    return values


def assert_activated_within_bounds(
    actual: torch.Tensor, x: torch.Tensor, w_gate_up: torch.Tensor, exact_fraction: float = 0.99,
    bias: torch.Tensor | None = None, **act
) -> None:
    """Activations within the interval their Gate / Up projections (plus the fp32 ``bias``
    [2 I] when given) allow, through the gated activation of ``act`` (function, alpha,
    limit, up_offset) at the payload rounding points, plus one ulp."""

    dtype = actual.dtype
    g_lo, g_hi = projection_interval(x, w_gate_up[0::2], dtype, None if bias is None else bias[0::2])
    u_lo, u_hi = projection_interval(x, w_gate_up[1::2], dtype, None if bias is None else bias[1::2])
    low = high = None
    for g in _candidates(g_lo, g_hi):
        for u in _candidates(u_lo, u_hi):
            h = _gated(g, u, dtype, **act).double()
            low = h if low is None else torch.minimum(low, h)
            high = h if high is None else torch.maximum(high, h)
    slack_low = _ulp(low.float(), dtype).double()
    slack_high = _ulp(high.float(), dtype).double()
    a = actual.detach().cpu()
    assert torch.isfinite(a.float()).all()
    value = a.double()
    outside = int(((value < low - slack_low) | (value > high + slack_high)).sum().item())
    assert outside == 0, f"{outside} of {a.numel()} activations outside their rounding-point interval"
    nominal = stage_activated(x, w_gate_up, dtype=dtype, bias=bias, **act)
    exact = float((a.view(torch.int16) == nominal.view(torch.int16)).float().mean())
    assert exact >= exact_fraction, f"only {exact:.4f} of activations are bit-identical to the oracle"


def assert_moe_stages(intermediates: dict, x, w_gate_up, w_down, ids, weights, output, scale: float = 1.0,
                      **act) -> None:
    """Each Experts stage against the oracle, fed with the GPU's own previous stage.

    * the sort: every live route appears once, grouped by expert, ``expert_end`` consistent;
    * activations within their fp32-accumulation intervals (assert_activated_within_bounds);
    * route outputs ``p(fp32(h . w_down[e]) * gamma)`` within the interval of the GPU's
      activations (widened by the fp32 product's rounding), p the payload rounding;
    * the combine ``p(scale * sum over slots in order of float(route))`` bit for bit.

    The payload dtype (bf16 or fp16) is the activations'.  ``act`` holds the activation
    (function, approximate, alpha, limit, up_offset) and the optional fp32 projection biases
    ``i_bias`` [E, 2I] and ``o_bias`` [E, H], added before their rounding points.
    """

    act = dict(act)
    i_bias = act.pop("i_bias", None)
    o_bias = act.pop("o_bias", None)

    rows, topk = ids.shape
    experts = w_gate_up.shape[0]
    flat_ids = ids.flatten()
    live = int(((flat_ids >= 0) & (flat_ids < experts)).sum())
    sorted_route = intermediates["sorted_route"].cpu().long()[:live]
    activated = intermediates["activated"].cpu()[:live]
    route_out = intermediates["route_out"].cpu()
    expert_end = intermediates["expert_end"].cpu().long()
    dtype = activated.dtype
    assert torch.equal(sorted_route.sort().values, torch.nonzero(flat_ids >= 0).flatten())
    experts_of = flat_ids[sorted_route]
    assert bool((experts_of[1:] >= experts_of[:-1]).all()), "routes are not grouped by expert"
    assert torch.equal(expert_end, torch.bincount(experts_of, minlength=experts).cumsum(0))
    by_route = torch.zeros((rows * topk, activated.shape[1]), dtype=dtype)
    by_route[sorted_route] = activated
    gammas = weights.flatten().double()
    identical = 0
    for expert in range(experts):
        q = torch.nonzero(flat_ids == expert).flatten()
        if q.numel() == 0:
            continue
        expert_bias = None if i_bias is None else i_bias[expert]
        assert_activated_within_bounds(by_route[q], x[q // topk], w_gate_up[expert], exact_fraction=0.0,
                                       bias=expert_bias, **act)
        nominal = stage_activated(x[q // topk], w_gate_up[expert], dtype=dtype, bias=expert_bias, **act)
        identical += int((by_route[q].view(torch.int16) == nominal.view(torch.int16)).sum())
        h = by_route[q].double()
        w = w_down[expert].double()
        exact = h @ w.t()
        delta = (h.abs() @ w.abs().t()) * ACCUMULATION_BOUND
        if o_bias is not None:
            exact = exact + o_bias[expert].double()
            delta = delta + (exact.abs() + delta) * 2.0**-23
        gamma = gammas[q].unsqueeze(1)
        low, high = (exact - delta) * gamma, (exact + delta) * gamma
        low = low - low.abs() * 2.0**-23
        high = high + high.abs() * 2.0**-23
        got = route_out[q].double()
        outside = int(((got < floor16(low, dtype).double()) | (got > ceil16(high, dtype).double())).sum())
        assert outside == 0, f"expert {expert}: {outside} route outputs outside their interval"
    assert identical >= 0.99 * live * activated.shape[1], "fewer than 99 % of activations match the oracle's bits"
    total = torch.zeros((rows, route_out.shape[1]), dtype=torch.float32)
    for slot in range(topk):
        valid = ((ids[:, slot] >= 0) & (ids[:, slot] < experts)).unsqueeze(1)
        routes = route_out[torch.arange(rows) * topk + slot].float()
        total = total + torch.where(valid, routes, torch.zeros_like(routes))
    assert_bitwise_equal(output, (total * torch.tensor(scale, dtype=torch.float32)).to(dtype))


def stage_activated(x: torch.Tensor, w_gate_up: torch.Tensor, dtype: torch.dtype = torch.bfloat16,
                    bias: torch.Tensor | None = None, **act) -> torch.Tensor:
    """Oracle gate_up (plus the fp32 ``bias`` when given) and gated activation with the
    reference's rounding points, in the payload ``dtype``."""

    projected = x.double() @ w_gate_up.double().t()
    if bias is not None:
        projected = projected + bias.double()
    return _gated(projected[:, 0::2].to(dtype), projected[:, 1::2].to(dtype), dtype, **act)


def to_device(tensor: torch.Tensor, device) -> torch.Tensor:
    return tensor.contiguous().to(device)


def slots_tensor(slots: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(slots, dtype=np.int32)).to(device)
