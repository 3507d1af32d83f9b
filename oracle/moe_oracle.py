"""torch-CPU restatement of the reference MoE Router, routing finalisation and Experts.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Paths are relative to the CrossPool
checkout:

* ``router_topk`` follows router_topk_kernel, src/xpool/runtime/ffnagent/operators/
  routing.py:21-89: fp32 softmax (ties to the lower id) or sigmoid (ties to the higher id),
  selection-only correction bias, a sigmoid selection over bf16 logits stored through the
  bf16 logits buffer, the selected score as weight, renormalisation by the positive sum,
  optional rounding of the weights to the logits dtype.  A per-slot loop, not torch.topk,
  so the tie policy is explicit.
* ``router_logits`` follows Router.run_into (routing.py:148-190): PAYLOAD rounds the
  projection to bf16, FP32 / FP32_LOGITS keep fp32 logits (fp64 sums rounded once).
* ``finalize_routing`` follows finalize_moe_routing_kernel (routing.py:193-227).
* ``experts_reference`` is the reference's own expected-value formula for Experts,
  tests/suites/integration/runtime/ffnagent/test_operators.py:255-281, with fp64 instead of
  fp32 matrix-vector products: projection rounded to the payload dtype (bf16 or fp16),
  activation in fp32 rounded to it, down projection times the route weight rounded to it,
  fp32 sum over the row's slots in order, times the routed scaling factor, rounded to it.
* ``experts_fp32`` is the same without any intermediate rounding (the pure-fp32 side of the
  parity bar).

Pinned in tests/test_moe_oracle.py by the known answers of the reference's routing tests
(routing/test_softmax_payload.py, test_softmax_fp32.py, test_sigmoid.py tie-policy case,
test_metadata.py), by torch.softmax / torch.topk / torch.sigmoid on tie-free inputs, by a
second, literal fp32 transcription of the reference's Experts formula on its own 4-expert
test case (which must stay within ``rounding_slack``), by the reduction to the Dense oracle
(one expert, one route, weight and scale 1: bit-identical), and by planted mistakes.
"""

from __future__ import annotations

import torch

from oracle import ffn_oracle as o


def router_logits(x: torch.Tensor, w: torch.Tensor, *, payload: bool, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """fp32 logits as the Router projection produces them (rounded to the payload ``dtype``,
    bf16 or fp16, for PAYLOAD)."""

    exact = x.double() @ w.double().t()
    return exact.to(dtype).float() if payload else exact.float()


def router_topk(
    logits: torch.Tensor,
    *,
    topk: int,
    softmax: bool,
    correction_bias: torch.Tensor | None = None,
    renormalize: bool = True,
    round_weights: bool = False,
    logits_bf16: bool = False,
    logits_dtype: torch.dtype | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """ids [rows, topk] int32 and weights [rows, topk] fp32 of router_topk_kernel.

    ``logits_dtype`` (or ``logits_bf16``) names the 16-bit dtype the logits are stored in,
    whose rounding the sigmoid selection and the LOGITS_DTYPE weight rounding take."""

    if logits_dtype is None and logits_bf16:
        logits_dtype = torch.bfloat16
    logits = logits.float()
    rows, experts = logits.shape
    if softmax:
        shifted = logits - logits.max(dim=1, keepdim=True).values
        exponentials = torch.exp(shifted)
        scores = exponentials / exponentials.sum(dim=1, keepdim=True)
    else:
        scores = torch.sigmoid(logits)
    selection = scores.clone()
    if correction_bias is not None:
        selection = selection + correction_bias.float()
    if not softmax and logits_dtype is not None:
        selection = selection.to(logits_dtype).float()
    ids = torch.empty((rows, topk), dtype=torch.int32)
    weights = torch.empty((rows, topk), dtype=torch.float32)
    for row in range(rows):
        remaining = selection[row].clone()
        normalizer = torch.zeros((), dtype=torch.float32)
        for slot in range(topk):
            maximum = remaining.max()
            tied = torch.nonzero(remaining == maximum).flatten()
            expert = int(tied.min()) if softmax else int(tied.max())
            weight = maximum if softmax and correction_bias is None else scores[row, expert]
            ids[row, slot] = expert
            weights[row, slot] = weight
            normalizer = normalizer + weight
            remaining[expert] = float("-inf")
        if renormalize:
            weights[row] = weights[row] / (normalizer if normalizer > 0 else torch.ones(()))
        if round_weights and logits_dtype is not None:
            weights[row] = weights[row].to(logits_dtype).float()
    return ids, weights


def finalize_routing(
    routed_ids: torch.Tensor,
    routed_weights: torch.Tensor,
    *,
    payload_rows: int,
    routed_expert_count: int,
    shared_expert_count: int,
    routed_scaling_factor: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Final Routing Metadata [capacity, routed_topk + shared] (routing.py:193-227)."""

    capacity, routed_topk = routed_ids.shape
    effective = routed_topk + shared_expert_count
    ids = torch.full((capacity, effective), -1, dtype=torch.int32)
    weights = torch.zeros((capacity, effective), dtype=torch.float32)
    live = min(payload_rows, capacity)
    ids[:live, :routed_topk] = routed_ids[:live]
    weights[:live, :routed_topk] = routed_weights[:live].float()
    for shared in range(shared_expert_count):
        ids[:live, routed_topk + shared] = routed_expert_count + shared
        weights[:live, routed_topk + shared] = torch.tensor(1.0 / routed_scaling_factor, dtype=torch.float32)
    return ids, weights


def _routes_by_expert(topk_ids: torch.Tensor, experts: int):
    rows, slots = topk_ids.shape
    for expert in range(experts):
        where = torch.nonzero(topk_ids == expert)
        if where.numel():
            yield expert, where[:, 0], where[:, 1]


def gated(gate: torch.Tensor, up: torch.Tensor, *, function: str = "silu", approximate: str = "none",
          alpha: float = 1.0, limit: float | None = None, up_offset: float = 0.0,
          dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """The Experts' gated activation of rounded Gate / Up values, rounded to ``dtype``:
    ``o.gated_silu`` for SiLU, ``o.gated_activation`` (compute_gated, activation.py:44-51)
    for ReLU and GELU."""

    if function == "silu":
        return o.gated_silu(gate, up, alpha=alpha, limit=limit, up_offset=up_offset, dtype=dtype)
    return o.gated_activation(gate, up, function=function, approximate=approximate, limit=limit,
                              up_offset=up_offset).to(dtype)


def experts_routes(
    x: torch.Tensor,
    w_gate_up: torch.Tensor,
    w_down: torch.Tensor,
    topk_ids: torch.Tensor,
    topk_weights: torch.Tensor,
    *,
    alpha: float = 1.0,
    limit: float | None = None,
    up_offset: float = 0.0,
    dtype: torch.dtype = torch.bfloat16,
    function: str = "silu",
    approximate: str = "none",
    i_bias: torch.Tensor | None = None,
    o_bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """Route outputs [rows, slots, hidden] (payload-dtype values held in fp32; 0 where no route).

    Projection plus its fp32 bias (``i_bias`` [E, 2I]) rounded to the payload ``dtype``
    (bf16 or fp16), activation (``function``: silu, relu or gelu) in fp32 rounded to it,
    down projection plus its bias (``o_bias`` [E, H]) times the route weight in fp32
    rounded to it (test_operators.py:255-278, where the reference runs the formula for each
    payload dtype, activation and bias case).
    """

    rows, hidden = x.shape
    experts = w_gate_up.shape[0]
    routes = torch.zeros((rows, topk_ids.shape[1], hidden), dtype=torch.float32)
    for expert, row_index, slot_index in _routes_by_expert(topk_ids, experts):
        projected = x[row_index].double() @ w_gate_up[expert].double().t()
        if i_bias is not None:
            projected = projected + i_bias[expert].double()
        projected = projected.to(dtype)
        activated = gated(projected[:, 0::2], projected[:, 1::2], function=function, approximate=approximate,
                          alpha=alpha, limit=limit, up_offset=up_offset, dtype=dtype)
        route = activated.double() @ w_down[expert].double().t()
        if o_bias is not None:
            route = route + o_bias[expert].double()
        gamma = topk_weights[row_index, slot_index].double().unsqueeze(1)
        routes[row_index, slot_index] = (route.float() * gamma.float()).to(dtype).float()
    return routes


def experts_reference(
    x: torch.Tensor,
    w_gate_up: torch.Tensor,
    w_down: torch.Tensor,
    topk_ids: torch.Tensor,
    topk_weights: torch.Tensor,
    *,
    routed_scaling_factor: float = 1.0,
    dtype: torch.dtype = torch.bfloat16,
    **act,
) -> torch.Tensor:
    """Expected Experts output with the reference's rounding points ([rows, hidden] of ``dtype``);
    ``act`` as :func:`experts_routes` takes it."""

    routes = experts_routes(x, w_gate_up, w_down, topk_ids, topk_weights, dtype=dtype, **act)
    total = torch.zeros(routes.shape[::2], dtype=torch.float32)
    for slot in range(topk_ids.shape[1]):
        total = total + routes[:, slot]
    return (total * routed_scaling_factor).to(dtype)


def rounding_slack(routes: torch.Tensor, expected: torch.Tensor, routed_scaling_factor: float = 1.0,
                   dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Per-element gap two correct implementations may show at the reference's rounding points.

    Each route output is rounded to the payload ``dtype`` before the sum, so an
    implementation whose fp32 accumulation differs may land one ulp away on every route; the
    scaled sum is then rounded once more: scale * sum_k ulp(r_k) + ulp(y).
    """

    ulp = o.bf16_ulp if dtype is torch.bfloat16 else o.f16_ulp
    route_ulps = ulp(routes.abs()) * (routes != 0)
    return routed_scaling_factor * route_ulps.sum(dim=1) + ulp(expected.float().abs())


def experts_fp32(
    x: torch.Tensor,
    w_gate_up: torch.Tensor,
    w_down: torch.Tensor,
    topk_ids: torch.Tensor,
    topk_weights: torch.Tensor,
    *,
    routed_scaling_factor: float = 1.0,
    alpha: float = 1.0,
    limit: float | None = None,
    up_offset: float = 0.0,
    function: str = "silu",
    approximate: str = "none",
    i_bias: torch.Tensor | None = None,
    o_bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """The same Experts output in fp32 with no intermediate rounding."""

    rows, hidden = x.shape
    experts = w_gate_up.shape[0]
    total = torch.zeros((rows, hidden), dtype=torch.float64)
    for expert, row_index, slot_index in _routes_by_expert(topk_ids, experts):
        projected = x[row_index].double() @ w_gate_up[expert].double().t()
        if i_bias is not None:
            projected = projected + i_bias[expert].double()
        gate, up = projected[:, 0::2], projected[:, 1::2]
        if limit is not None:
            gate = torch.clamp(gate, max=limit)
            up = torch.clamp(up, -limit, limit)
        if function == "silu":
            activated = gate * torch.sigmoid(alpha * gate) * (up + up_offset)
        else:
            activated = o.activation_function(gate, function, approximate=approximate).double() * (up + up_offset)
        route = activated @ w_down[expert].double().t()
        if o_bias is not None:
            route = route + o_bias[expert].double()
        total.index_add_(0, row_index, route * topk_weights[row_index, slot_index].double().unsqueeze(1))
    return (total * routed_scaling_factor).float()


def generate_moe_layer(hidden: int, intermediate: int, experts: int, seed: int, std: float = 0.02,
                       dtype: torch.dtype = torch.bfloat16):
    """Seeded Expert weights of ``dtype``: i_proj [E, 2I, H] (interleaved), o_proj [E, H, I]."""

    generator = torch.Generator().manual_seed(seed)
    w_gate_up = (torch.randn((experts, 2 * intermediate, hidden), generator=generator) * std).to(dtype)
    w_down = (torch.randn((experts, hidden, intermediate), generator=generator) * std).to(dtype)
    return w_gate_up, w_down


def generate_routes(rows: int, experts: int, topk: int, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Seeded distinct expert ids per row and positive weights summing to one."""

    generator = torch.Generator().manual_seed(seed)
    scores = torch.rand((rows, experts), generator=generator)
    ids = torch.argsort(scores, dim=1, descending=True)[:, :topk].to(torch.int32)
    weights = torch.rand((rows, topk), generator=generator) + 0.05
    return ids, (weights / weights.sum(dim=1, keepdim=True)).float()
