"""GPU parity of the MoE Router, routing finalisation and Experts against oracle/moe_oracle.py.

Router cases are the reference's own routing tests (routing/test_softmax_payload.py,
test_softmax_fp32.py, test_sigmoid.py, test_metadata.py), with bf16 and fp16 payloads as
those tests parametrize them: ids must match exactly and weights within rtol 1e-5 /
atol 1e-6, the reference's tolerance.  On random Qwen3-MoE-shaped
inputs the projection's bf16 logits must lie in their fp32-accumulation intervals and the
TopK over those logits must match the oracle's TopK on the same logits.  Experts outputs meet
the MoE bar of tests/parity.py against the reference's expected-value formula
(test_operators.py:255-281) and its pure-fp32 counterpart, every stage (sort, activations,
route outputs, combine) is checked rigorously on the GPU's own intermediates, and outputs
repeat bit for bit.  fp16 Experts (test_operators.py:114) run on every grouped kernel
family with fp16 rounding points in the oracle.  As in the reference's routing and operator
tests, the Router and Experts are captured into graphs without allocation and replayed over
inputs changed in place, each replay checked against the oracle and an eager call.
"""

from __future__ import annotations

import pytest
import torch

from crosspool_amd.ffn import GateTransform, GeluActivation, ReluActivation, RouterAlgorithm, RouterProjectionPrecision
from crosspool_amd.ffn import SiluActivation
from crosspool_amd.ffn import TopKWeightRounding
from crosspool_amd.moe import Experts, MoeFfnWeights, MoeRouterWeights, Router, finalize_moe_routing, router_topk
from oracle import ffn_oracle as o
from oracle import moe_oracle as m
from parity import assert_bitwise_equal, assert_moe_parity, assert_moe_stages, assert_projection_within_bounds
from parity import stage_activated, to_device

pytestmark = pytest.mark.gpu

TWO_ROWS = ((3.0, 1.0, -1.0, -3.0), (-2.0, 0.0, 2.0, 4.0))
PAYLOADS = pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16), ids=("bfloat16", "float16"))


def _router(device, hidden_states, projection, **kwargs):
    rows, hidden = hidden_states.shape
    router = Router(row_capacity=rows, hidden_size=hidden, routed_expert_count=projection.shape[0], device=device,
                    **kwargs)
    return router


@PAYLOADS
@pytest.mark.parametrize("rounding", tuple(TopKWeightRounding))
def test_softmax_payload_router(device, rounding, dtype):
    # routing/test_softmax_payload.py:16-60
    hidden = torch.tensor(TWO_ROWS, dtype=dtype)
    projection = torch.eye(4, dtype=dtype)
    router = _router(device, hidden, projection, routed_topk=2, algorithm=RouterAlgorithm.SOFTMAX,
                     precision=RouterProjectionPrecision.PAYLOAD, renormalize=True, weight_rounding=rounding,
                     payload_dtype=dtype)
    router.run_into(hidden_states=to_device(hidden, device), router_weights=MoeRouterWeights(to_device(projection, device)))
    assert router.logits.dtype is dtype
    ids, weights = m.router_topk(m.router_logits(hidden, projection, payload=True, dtype=dtype), topk=2, softmax=True,
                                 round_weights=rounding is TopKWeightRounding.LOGITS_DTYPE, logits_dtype=dtype)
    assert torch.equal(router.ids.cpu(), ids) and ids.tolist() == [[0, 1], [3, 2]]
    torch.testing.assert_close(router.weights.cpu(), weights, rtol=1e-5, atol=1e-6)


@PAYLOADS
@pytest.mark.parametrize("corrected", (False, True))
def test_softmax_fp32_logits_router_with_correction(device, corrected, dtype):
    # routing/test_softmax_fp32.py:15-60
    hidden = torch.tensor(TWO_ROWS, dtype=dtype)
    projection = torch.eye(4, dtype=dtype)
    bias = torch.tensor((-0.75, -0.25, 0.5, 0.8)) if corrected else None
    router = _router(device, hidden, projection, routed_topk=2, algorithm=RouterAlgorithm.SOFTMAX,
                     precision=RouterProjectionPrecision.FP32_LOGITS, renormalize=False, payload_dtype=dtype)
    weights_gpu = MoeRouterWeights(to_device(projection, device), None if bias is None else to_device(bias, device))
    router.run_into(hidden_states=to_device(hidden, device), router_weights=weights_gpu)
    ids, weights = m.router_topk(m.router_logits(hidden, projection, payload=False), topk=2, softmax=True,
                                 correction_bias=bias, renormalize=False)
    assert torch.equal(router.ids.cpu(), ids)
    torch.testing.assert_close(router.weights.cpu(), weights, rtol=1e-5, atol=1e-6)


@PAYLOADS
@pytest.mark.parametrize("experts,topk,scale", ((64, 4, 4096.0), (48, 3, None), (17, 1, 1.0), (17, 17, 1.0)))
def test_sigmoid_fp32_router_diagonal(device, experts, topk, scale, dtype):
    # routing/test_sigmoid.py:15-73
    hidden = (torch.arange(2 * experts, dtype=torch.float32).view(2, experts) / (2 * experts)).to(dtype)
    bias = torch.linspace(-0.25, 0.25, experts) * scale if scale is not None else None
    projection = torch.diag(torch.linspace(0.101, 1.909, experts))
    router = _router(device, hidden, projection, routed_topk=topk, algorithm=RouterAlgorithm.SIGMOID,
                     precision=RouterProjectionPrecision.FP32, renormalize=True, payload_dtype=dtype)
    weights_gpu = MoeRouterWeights(to_device(projection, device), None if bias is None else to_device(bias, device))
    router.run_into(hidden_states=to_device(hidden, device), router_weights=weights_gpu)
    ids, weights = m.router_topk(m.router_logits(hidden, projection, payload=False), topk=topk, softmax=False,
                                 correction_bias=bias, renormalize=True)
    assert torch.equal(router.ids.cpu(), ids)
    torch.testing.assert_close(router.weights.cpu(), weights, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("algorithm", (RouterAlgorithm.SOFTMAX, RouterAlgorithm.SIGMOID))
def test_router_tie_policy(device, algorithm):
    # routing/test_sigmoid.py:76-117
    hidden = torch.tensor(((0.0,) * 17, (-1000.0,) * 17), dtype=torch.bfloat16)
    softmax = algorithm is RouterAlgorithm.SOFTMAX
    precision = RouterProjectionPrecision.PAYLOAD if softmax else RouterProjectionPrecision.FP32
    projection = torch.eye(17, dtype=torch.bfloat16 if softmax else torch.float32)
    router = _router(device, hidden, projection, routed_topk=3, algorithm=algorithm, precision=precision,
                     renormalize=True)
    router.run_into(hidden_states=to_device(hidden, device), router_weights=MoeRouterWeights(to_device(projection, device)))
    expected_ids = (0, 1, 2) if softmax else (16, 15, 14)
    second = (1 / 3, 1 / 3, 1 / 3) if softmax else (0.0, 0.0, 0.0)
    assert router.ids.cpu().tolist() == [list(expected_ids)] * 2
    torch.testing.assert_close(router.weights.cpu(), torch.tensor(((1 / 3, 1 / 3, 1 / 3), second)), rtol=1e-5,
                               atol=1e-6)


@PAYLOADS
@pytest.mark.parametrize("rows", (1, 16, 200))
def test_qwen3_moe_router_projection_and_topk(device, rows, dtype):
    # Qwen3-30B-A3B router: 128 experts over hidden 2048, top-8, softmax, renormalised.
    hidden, experts = 2048, 128
    x = o.generate_hidden_states(rows, hidden, 70 + rows).to(dtype)
    generator = torch.Generator().manual_seed(71)
    projection = (torch.randn((experts, hidden), generator=generator) * 0.02).to(dtype)
    router = Router(row_capacity=rows, hidden_size=hidden, routed_expert_count=experts, routed_topk=8, device=device,
                    payload_dtype=dtype)
    router.run_into(hidden_states=to_device(x, device), router_weights=MoeRouterWeights(to_device(projection, device)))
    logits = router.logits.cpu()
    assert logits.dtype is dtype
    assert_projection_within_bounds(logits, x, projection)
    ids, weights = m.router_topk(logits.float(), topk=8, softmax=True, logits_dtype=dtype)
    assert torch.equal(router.ids.cpu(), ids)
    torch.testing.assert_close(router.weights.cpu(), weights, rtol=1e-5, atol=1e-6)
    # TopK alone over the same logits.
    ids_only, weights_only = router_topk(router.logits, topk=8, algorithm=RouterAlgorithm.SOFTMAX)
    assert torch.equal(ids_only.cpu(), ids)
    torch.testing.assert_close(weights_only.cpu(), weights, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("softmax", (True, False), ids=("softmax", "sigmoid"))
@pytest.mark.parametrize("experts", (17, 128, 129, 256, 300, 512, 700, 1024))
def test_topk_at_every_expert_width(device, experts, softmax):
    # The TopK kernel holds 2, 4, 8 or 16 experts per lane (the fewest that cover the count:
    # 128 / 256 / 512 / 1024 experts), each width its own instantiation.  Logits on a grid of
    # eighths make ties common, also between experts that sit in different slots of one lane,
    # so the tie policy (lower id for softmax, higher for sigmoid) is checked at every width.
    rows, topk = 37, 8
    generator = torch.Generator().manual_seed(500 + experts)
    logits = torch.randint(-24, 25, (rows, experts), generator=generator).float() / 8
    bias = None if softmax else torch.randint(-4, 5, (experts,), generator=generator).float() / 16
    algorithm = RouterAlgorithm.SOFTMAX if softmax else RouterAlgorithm.SIGMOID
    ids, weights = router_topk(to_device(logits, device), topk=topk, algorithm=algorithm,
                               correction_bias=None if bias is None else to_device(bias, device))
    expected_ids, expected_weights = m.router_topk(logits, topk=topk, softmax=softmax, correction_bias=bias)
    assert torch.equal(ids.cpu(), expected_ids)
    torch.testing.assert_close(weights.cpu(), expected_weights, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("softmax", (True, False), ids=("softmax", "sigmoid"))
@pytest.mark.parametrize("experts", (17, 128, 300))
def test_topk_over_fp16_logits(device, experts, softmax):
    # fp16 logits (an fp16 layer's PAYLOAD projection): the sigmoid selection is rounded to
    # fp16, as the LOGITS_DTYPE weight rounding is; values on a grid of sixteenths keep ties.
    rows, topk = 29, 6
    generator = torch.Generator().manual_seed(600 + experts)
    logits = (torch.randint(-48, 49, (rows, experts), generator=generator).float() / 16).half()
    bias = None if softmax else torch.randint(-4, 5, (experts,), generator=generator).float() / 1024
    algorithm = RouterAlgorithm.SOFTMAX if softmax else RouterAlgorithm.SIGMOID
    for rounding in tuple(TopKWeightRounding):
        ids, weights = router_topk(to_device(logits, device), topk=topk, algorithm=algorithm,
                                   correction_bias=None if bias is None else to_device(bias, device),
                                   weight_rounding=rounding)
        expected_ids, expected_weights = m.router_topk(
            logits.float(), topk=topk, softmax=softmax, correction_bias=bias, logits_dtype=torch.float16,
            round_weights=rounding is TopKWeightRounding.LOGITS_DTYPE)
        assert torch.equal(ids.cpu(), expected_ids)
        torch.testing.assert_close(weights.cpu(), expected_weights, rtol=1e-5, atol=1e-6)


def test_finalize_routing_dynamic_live_rows(device):
    # routing/test_metadata.py:8-80
    routed_ids = torch.tensor(((0, 2), (1, 3), (2, 0), (3, 1)), dtype=torch.int32, device=device)
    routed_weights = torch.tensor(((0.75, 0.25), (0.6, 0.4), (0.9, 0.1), (0.55, 0.45)), device=device)
    final_ids = torch.empty((4, 3), dtype=torch.int32, device=device)
    final_weights = torch.empty((4, 3), dtype=torch.float32, device=device)
    payload_rows = torch.tensor((2,), dtype=torch.int64, device=device)
    kwargs = dict(routed_expert_count=4, shared_expert_count=1, routed_scaling_factor=2.0)
    for live in (2, 3):
        payload_rows.fill_(live)
        finalize_moe_routing(routed_ids=routed_ids, routed_weights=routed_weights, final_ids=final_ids,
                             final_weights=final_weights, payload_rows=payload_rows, **kwargs)
        ids, weights = m.finalize_routing(routed_ids.cpu(), routed_weights.cpu(), payload_rows=live, **kwargs)
        assert torch.equal(final_ids.cpu(), ids)
        torch.testing.assert_close(final_weights.cpu(), weights, rtol=0, atol=0)
    assert final_ids.cpu()[:2].tolist() == [[0, 2, 4], [1, 3, 4]]


def _run_experts(device, x, w_gate_up, w_down, ids, weights, scale=1.0, activation=None, gate=None, i_bias=None,
                 o_bias=None):
    rows, hidden = x.shape
    experts, two_i, _ = w_gate_up.shape
    operator = Experts(row_capacity=rows, hidden_size=hidden, local_intermediate_size=two_i // 2,
                       expert_count=experts, effective_topk=ids.shape[1], routed_scaling_factor=scale,
                       activation=activation, gate=gate, device=device, payload_dtype=x.dtype)
    weights_gpu = MoeFfnWeights(to_device(w_gate_up, device), to_device(w_down, device),
                                i_proj_bias=None if i_bias is None else to_device(i_bias, device),
                                o_proj_bias=None if o_bias is None else to_device(o_bias, device))
    output = torch.empty((rows, hidden), dtype=x.dtype, device=device)
    operator.run_into(hidden_states=to_device(x, device), weights=weights_gpu, topk_ids=to_device(ids, device),
                      topk_weights=to_device(weights, device), output=output)
    return output.cpu(), operator, weights_gpu


def _check_experts(got, x, w_gate_up, w_down, ids, weights, scale=1.0, **act):
    dtype = x.dtype
    assert got.dtype is dtype
    routes = m.experts_routes(x, w_gate_up, w_down, ids, weights, dtype=dtype, **act)
    stage = m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=scale, dtype=dtype, **act)
    pure = m.experts_fp32(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=scale, **act)
    assert_moe_parity(got, stage, pure, m.rounding_slack(routes, stage, scale, dtype=dtype))


def _activation_of(act):
    function = act.get("function", "silu")
    if function == "relu":
        return ReluActivation()
    if function == "gelu":
        return GeluActivation(act.get("approximate", "none"))
    return SiluActivation(act.get("alpha", 1.0))


# test_operators.py:110-121: payload dtype, projection biases, activation and gate transform.
OPERATOR_CASES = [
    pytest.param(torch.bfloat16, False, {}, id="bf16-silu"),
    pytest.param(torch.float16, False, {}, id="fp16-silu"),
    pytest.param(torch.bfloat16, True, {}, id="bf16-bias-silu"),
    pytest.param(torch.bfloat16, True, {"alpha": 1.702, "limit": 7.0, "up_offset": 1.0}, id="bf16-bias-swiglu"),
    pytest.param(torch.bfloat16, False, {"alpha": 1.702, "limit": 7.0, "up_offset": 1.0}, id="bf16-swiglu"),
    pytest.param(torch.bfloat16, True, {"function": "relu", "limit": 4.0, "up_offset": -0.5}, id="bf16-bias-relu"),
    pytest.param(torch.bfloat16, True, {"function": "gelu"}, id="bf16-bias-gelu"),
    pytest.param(torch.bfloat16, True, {"function": "gelu", "approximate": "tanh"}, id="bf16-bias-gelu-tanh"),
]


@pytest.mark.parametrize("dtype,with_bias,act", OPERATOR_CASES)
def test_experts_reference_operator_case(device, dtype, with_bias, act):
    # test_operators.py:110-281: four experts, two slots, a dead row, scale 1.5, every
    # payload / bias / activation case of the reference's parametrization.
    generator = torch.Generator().manual_seed(31)
    x = (torch.randn((4, 16), generator=generator) / 4).to(dtype)
    w_gate_up = (torch.randn((4, 16, 16), generator=generator) / 4).to(dtype)
    w_down = (torch.randn((4, 16, 8), generator=generator) / 4).to(dtype)
    ids = torch.tensor(((0, 1), (2, 3), (1, 3), (-1, -1)), dtype=torch.int32)
    weights = torch.tensor(((0.75, 0.25), (0.6, 0.4), (0.9, 0.1), (0.0, 0.0)))
    if with_bias:
        bias_generator = torch.Generator().manual_seed(32)
        act = {**act, "i_bias": torch.randn((4, 16), generator=bias_generator),
               "o_bias": torch.randn((4, 16), generator=bias_generator)}
    gate = GateTransform(limit=act.get("limit"), up_offset=act.get("up_offset", 0.0))
    got, operator, _ = _run_experts(device, x, w_gate_up, w_down, ids, weights, 1.5, _activation_of(act), gate,
                                    act.get("i_bias"), act.get("o_bias"))
    assert_moe_stages(operator.intermediates(), x, w_gate_up, w_down, ids, weights, got, 1.5, **act)
    stage = m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5, dtype=dtype, **act)
    routes = m.experts_routes(x, w_gate_up, w_down, ids, weights, dtype=dtype, **act)
    assert got.dtype is dtype
    torch.testing.assert_close(got, stage, rtol=0.02, atol=0.1)
    gap = (got.float() - stage.float()).abs()
    assert (gap <= m.rounding_slack(routes, stage, 1.5, dtype=dtype)).all()
    assert o.compare(stage, got).normalized_rmse <= 0.01
    assert got[3].abs().sum() == 0


@pytest.mark.parametrize("rows", (1, 7, 48, 320))
def test_experts_qwen3_moe_shape(device, rows):
    # Qwen3-30B-A3B expert layer: hidden 2048, moe_intermediate 768, 128 experts, top-8.
    # 320 rows (20 routes per expert on average) take the grouped tile kernel on 64-row
    # expert tiles.
    hidden, intermediate, experts, topk = 2048, 768, 128, 8
    w_gate_up, w_down = m.generate_moe_layer(hidden, intermediate, experts, 90)
    x = o.generate_hidden_states(rows, hidden, 91 + rows)
    ids, weights = m.generate_routes(rows, experts, topk, 92 + rows)
    got, operator, weights_gpu = _run_experts(device, x, w_gate_up, w_down, ids, weights)
    _check_experts(got, x, w_gate_up, w_down, ids, weights)
    assert_moe_stages(operator.intermediates(), x, w_gate_up, w_down, ids, weights, got)
    again = torch.empty((rows, hidden), dtype=torch.bfloat16, device=device)
    operator.run_into(hidden_states=to_device(x, device), weights=weights_gpu, topk_ids=to_device(ids, device),
                      topk_weights=to_device(weights, device), output=again)
    assert_bitwise_equal(again.cpu(), got)


@pytest.mark.parametrize("rows", (96, 240, 480, 1024))
def test_experts_large_tiles_with_dead_rows(device, rows):
    # The grouped tile kernel (more than 4 routes per expert on average) at every expert tile
    # height: 24 routes per expert on 64-row tiles (96 rows), 60 on 128-row tiles with
    # nontemporal weight loads (240), 120 on 128-row tiles with plain loads (480), 256 on
    # 256-row tiles (1024); several tiles per expert, ragged tails, and a band of rows
    # without routes.
    hidden, intermediate, experts, topk = 256, 128, 8, 2
    w_gate_up, w_down = m.generate_moe_layer(hidden, intermediate, experts, 93, std=0.1)
    x = o.generate_hidden_states(rows, hidden, 94)
    ids, weights = m.generate_routes(rows, experts, topk, 95)
    ids[rows // 3: rows // 3 + 5] = -1
    weights[rows // 3: rows // 3 + 5] = 0.0
    got, operator, _ = _run_experts(device, x, w_gate_up, w_down, ids, weights, scale=2.5)
    _check_experts(got, x, w_gate_up, w_down, ids, weights, scale=2.5)
    assert_moe_stages(operator.intermediates(), x, w_gate_up, w_down, ids, weights, got, 2.5)
    assert got[rows // 3: rows // 3 + 5].abs().sum() == 0


@pytest.mark.parametrize("hidden,intermediate", ((512, 192), (1000, 264)))
def test_experts_decode_tiles_skewed_routing(device, hidden, intermediate):
    # Few routes per expert on average (16-route tiles of the grouped split kernel), but
    # slot 0 of every row goes to expert 3: that expert spans several tiles, the last one
    # ragged, while the others hold one or two routes.  1000 / 264 make the K ranges end
    # inside a 128-wide chunk.
    rows, experts, topk = 45, 24, 2
    w_gate_up, w_down = m.generate_moe_layer(hidden, intermediate, experts, 99, std=0.05)
    x = o.generate_hidden_states(rows, hidden, 100)
    ids, weights = m.generate_routes(rows, experts, topk, 101)
    ids[:, 0] = 3
    ids[:, 1] = torch.where(ids[:, 1] == 3, torch.full_like(ids[:, 1], 5), ids[:, 1])
    assert rows * topk <= 4 * experts and int((ids == 3).sum()) > 2 * 16
    got, operator, weights_gpu = _run_experts(device, x, w_gate_up, w_down, ids, weights, scale=1.25)
    _check_experts(got, x, w_gate_up, w_down, ids, weights, scale=1.25)
    assert_moe_stages(operator.intermediates(), x, w_gate_up, w_down, ids, weights, got, 1.25)
    again = torch.empty((rows, hidden), dtype=torch.bfloat16, device=device)
    operator.run_into(hidden_states=to_device(x, device), weights=weights_gpu, topk_ids=to_device(ids, device),
                      topk_weights=to_device(weights, device), output=again)
    assert_bitwise_equal(again.cpu(), got)


@pytest.mark.parametrize(
    "rows,hidden,intermediate,experts,topk",
    (
        (1, 2048, 768, 128, 8),     # grouped split, one route per expert
        (48, 2048, 768, 128, 8),    # grouped split, 16-route tiles
        (320, 2048, 768, 128, 8),   # 64-row grouped tiles
        (240, 256, 128, 8, 2),      # 128-row grouped tiles, nontemporal weight loads
        (480, 256, 128, 8, 2),      # 128-row grouped tiles
        (1024, 256, 128, 8, 2),     # 256-row grouped tiles
    ),
)
def test_experts_fp16_every_tile_family(device, rows, hidden, intermediate, experts, topk):
    # fp16 payloads (test_operators.py:114) through each grouped kernel the chooser takes,
    # with fp16 rounding points in the oracle and every stage checked.  Weights are drawn in
    # fp32 and stored in fp16, as an fp16 checkpoint holds them.
    w_gate_up, w_down = m.generate_moe_layer(hidden, intermediate, experts, 140 + rows, std=0.05,
                                             dtype=torch.float16)
    x = o.generate_hidden_states(rows, hidden, 141 + rows).half()
    ids, weights = m.generate_routes(rows, experts, topk, 142 + rows)
    ids[rows // 2: rows // 2 + rows // 8] = -1
    weights[rows // 2: rows // 2 + rows // 8] = 0.0
    got, operator, weights_gpu = _run_experts(device, x, w_gate_up, w_down, ids, weights, scale=1.25)
    _check_experts(got, x, w_gate_up, w_down, ids, weights, scale=1.25)
    assert_moe_stages(operator.intermediates(), x, w_gate_up, w_down, ids, weights, got, 1.25)
    again = torch.empty((rows, hidden), dtype=torch.float16, device=device)
    operator.run_into(hidden_states=to_device(x, device), weights=weights_gpu, topk_ids=to_device(ids, device),
                      topk_weights=to_device(weights, device), output=again)
    assert_bitwise_equal(again.cpu(), got)


@PAYLOADS
def test_experts_rows_independent_of_their_tile_position(device, dtype):
    # Every route carries the same token row to the same expert (640 routes: ten 64-row
    # tiles), so every tile row must store the same activations and every output row the same
    # bits.  The token / expert pair holds an exact fp16 tie: at column 442 the fp32 product
    # silu(g) * u lies on the midpoint of two fp16 values, and the reference rounds it to fp32
    # first and then to fp16 (to even).  A multiply fused into the fp16 conversion rounds the
    # exact product once and lands one ulp higher, in some unrolled epilogue slots only.
    rows, hidden, intermediate, experts = 640, 2048, 768, 128
    w_gate_up, w_down = m.generate_moe_layer(hidden, intermediate, experts, 460, std=0.05, dtype=dtype)
    token = o.generate_hidden_states(320, hidden, 461).to(dtype)[264]
    x = token.unsqueeze(0).repeat(rows, 1).contiguous()
    ids = torch.full((rows, 1), 103, dtype=torch.int32)
    weights = torch.ones((rows, 1))
    got, operator, _ = _run_experts(device, x, w_gate_up, w_down, ids, weights)
    activated = operator.intermediates()["activated"][:rows].cpu()
    bits = activated.view(torch.int16)
    assert bool((bits == bits[0]).all()), "a route's activations depend on its row in the expert tile"
    nominal = stage_activated(token.unsqueeze(0), w_gate_up[103], dtype=dtype)[0]
    if dtype is torch.float16:
        assert float(activated[0, 442]) == float(nominal[442]) == 2.11328125
    out = got.view(torch.int16)
    assert bool((out == out[0]).all())
    _check_experts(got, x, w_gate_up, w_down, ids, weights)


def _capture_no_alloc(run):
    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        before = torch.cuda.memory_stats()["allocation.all.allocated"]
        run()
        after = torch.cuda.memory_stats()["allocation.all.allocated"]
    assert before == after, "capture allocated memory"
    return graph


@PAYLOADS
@pytest.mark.parametrize("experts,topk,scale", ((64, 4, 4096.0), (17, 17, 1.0)))
def test_sigmoid_router_graph_replay_with_new_inputs(device, experts, topk, scale, dtype):
    # routing/test_sigmoid.py:48-73: the Router captured into a graph (no allocation), then
    # the hidden states halved and the correction negated in place before each replay.  Every
    # replay matches the oracle on the new inputs and an eager call on the same inputs.
    hidden = (torch.arange(2 * experts, dtype=torch.float32).view(2, experts) / (2 * experts)).to(dtype)
    projection = torch.diag(torch.linspace(0.101, 1.909, experts))
    router = _router(device, hidden, projection, routed_topk=topk, algorithm=RouterAlgorithm.SIGMOID,
                     precision=RouterProjectionPrecision.FP32, renormalize=True, payload_dtype=dtype)
    hidden_gpu = to_device(hidden, device)
    weights_gpu = MoeRouterWeights(to_device(projection, device),
                                   to_device(torch.linspace(-0.25, 0.25, experts) * scale, device))
    graph = _capture_no_alloc(lambda: router.run_into(hidden_states=hidden_gpu, router_weights=weights_gpu))
    for _ in range(3):
        hidden_gpu.mul_(0.5)
        weights_gpu.correction_bias.neg_()
        graph.replay()
        torch.cuda.synchronize()
        got_ids, got_weights = router.ids.cpu(), router.weights.cpu()
        ids, weights = m.router_topk(m.router_logits(hidden_gpu.cpu(), projection, payload=False), topk=topk,
                                     softmax=False, correction_bias=weights_gpu.correction_bias.cpu(),
                                     renormalize=True)
        assert torch.equal(got_ids, ids)
        torch.testing.assert_close(got_weights, weights, rtol=1e-5, atol=1e-6)
        router.run_into(hidden_states=hidden_gpu, router_weights=weights_gpu)
        torch.cuda.synchronize()
        assert torch.equal(router.ids.cpu(), got_ids) and torch.equal(router.weights.cpu(), got_weights)


@PAYLOADS
@pytest.mark.parametrize("rows", (1, 16, 200))
def test_qwen3_router_graph_replay_with_new_inputs(device, rows, dtype):
    # The PAYLOAD Router on the MFMA projection (K-slice sums in the TopK at decode sizes)
    # captured once and replayed over new token rows.
    hidden, experts = 2048, 128
    generator = torch.Generator().manual_seed(72)
    projection = (torch.randn((experts, hidden), generator=generator) * 0.02).to(dtype)
    router = Router(row_capacity=rows, hidden_size=hidden, routed_expert_count=experts, routed_topk=8, device=device,
                    payload_dtype=dtype)
    x_gpu = to_device(o.generate_hidden_states(rows, hidden, 73).to(dtype), device)
    weights_gpu = MoeRouterWeights(to_device(projection, device))
    graph = _capture_no_alloc(lambda: router.run_into(hidden_states=x_gpu, router_weights=weights_gpu))
    for step in range(3):
        x = o.generate_hidden_states(rows, hidden, 74 + step).to(dtype)
        x_gpu.copy_(to_device(x, device))
        graph.replay()
        torch.cuda.synchronize()
        got_ids, got_weights, got_logits = router.ids.cpu(), router.weights.cpu(), router.logits.cpu()
        assert_projection_within_bounds(got_logits, x, projection)
        ids, weights = m.router_topk(got_logits.float(), topk=8, softmax=True, logits_dtype=dtype)
        assert torch.equal(got_ids, ids)
        torch.testing.assert_close(got_weights, weights, rtol=1e-5, atol=1e-6)
        router.run_into(hidden_states=x_gpu, router_weights=weights_gpu)
        torch.cuda.synchronize()
        assert torch.equal(router.ids.cpu(), got_ids) and torch.equal(router.weights.cpu(), got_weights)
        assert_bitwise_equal(router.logits.cpu(), got_logits)


@PAYLOADS
def test_experts_graph_replay_with_new_inputs(device, dtype):
    # test_operators.py:234-281: the Experts operator captured without allocation, the
    # hidden states refilled with 3 before the replay, the output against the reference's
    # formula on the new inputs (its tolerance and the rounding-point slack), and the replay
    # equal to an eager call.
    generator = torch.Generator().manual_seed(31)
    x = (torch.randn((4, 16), generator=generator) / 4).to(dtype)
    w_gate_up = (torch.randn((4, 16, 16), generator=generator) / 4).to(dtype)
    w_down = (torch.randn((4, 16, 8), generator=generator) / 4).to(dtype)
    ids = torch.tensor(((0, 1), (2, 3), (1, 3), (-1, -1)), dtype=torch.int32)
    weights = torch.tensor(((0.75, 0.25), (0.6, 0.4), (0.9, 0.1), (0.0, 0.0)))
    operator = Experts(row_capacity=4, hidden_size=16, local_intermediate_size=8, expert_count=4, effective_topk=2,
                       routed_scaling_factor=1.5, device=device, payload_dtype=dtype)
    x_gpu = to_device(x, device)
    layer = MoeFfnWeights(to_device(w_gate_up, device), to_device(w_down, device))
    ids_gpu, weights_gpu = to_device(ids, device), to_device(weights, device)
    output = torch.empty_like(x_gpu)
    run = lambda: operator.run_into(hidden_states=x_gpu, weights=layer, topk_ids=ids_gpu, topk_weights=weights_gpu,
                                    output=output)  # noqa: E731
    graph = _capture_no_alloc(run)
    for fill in (3.0, -0.5):
        x_gpu.fill_(fill)
        graph.replay()
        torch.cuda.synchronize()
        got = output.cpu()
        new_x = x_gpu.cpu()
        stage = m.experts_reference(new_x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5, dtype=dtype)
        routes = m.experts_routes(new_x, w_gate_up, w_down, ids, weights, dtype=dtype)
        torch.testing.assert_close(got, stage, rtol=0.02, atol=0.1)
        assert ((got.float() - stage.float()).abs() <= m.rounding_slack(routes, stage, 1.5, dtype=dtype)).all()
        assert got[3].abs().sum() == 0
        run()
        torch.cuda.synchronize()
        assert_bitwise_equal(output.cpu(), got)


@PAYLOADS
@pytest.mark.parametrize("rows", (48, 320))
def test_experts_graph_replay_with_new_routing(device, rows, dtype):
    # Qwen3-30B-A3B experts captured once (grouped split kernel at 48 rows, grouped tiles at
    # 320) and replayed over new token rows and new routing: the route sort and tile table
    # are built on the device, so each replay serves its own routing.
    hidden, intermediate, experts, topk = 2048, 768, 128, 8
    w_gate_up, w_down = m.generate_moe_layer(hidden, intermediate, experts, 150, dtype=dtype)
    operator = Experts(row_capacity=rows, hidden_size=hidden, local_intermediate_size=intermediate,
                       expert_count=experts, effective_topk=topk, device=device, payload_dtype=dtype)
    layer = MoeFfnWeights(to_device(w_gate_up, device), to_device(w_down, device))
    first_ids, first_weights = m.generate_routes(rows, experts, topk, 151)
    x_gpu = to_device(o.generate_hidden_states(rows, hidden, 152).to(dtype), device)
    ids_gpu, weights_gpu = to_device(first_ids, device), to_device(first_weights, device)
    output = torch.empty_like(x_gpu)
    run = lambda: operator.run_into(hidden_states=x_gpu, weights=layer, topk_ids=ids_gpu, topk_weights=weights_gpu,
                                    output=output)  # noqa: E731
    graph = _capture_no_alloc(run)
    for step in range(2):
        x = o.generate_hidden_states(rows, hidden, 153 + step).to(dtype)
        ids, weights = m.generate_routes(rows, experts, topk, 155 + step)
        x_gpu.copy_(to_device(x, device))
        ids_gpu.copy_(to_device(ids, device))
        weights_gpu.copy_(to_device(weights, device))
        graph.replay()
        torch.cuda.synchronize()
        got = output.cpu()
        _check_experts(got, x, w_gate_up, w_down, ids, weights)
        run()
        torch.cuda.synchronize()
        assert_bitwise_equal(output.cpu(), got)


@pytest.mark.parametrize(
    "rows,hidden,intermediate,experts,topk",
    (
        (1, 2048, 768, 128, 8),     # grouped split
        (48, 2048, 768, 128, 8),    # grouped split, 16-route tiles
        (320, 2048, 768, 128, 8),   # 64-row grouped tiles
        (240, 256, 128, 8, 2),      # 128-row grouped tiles, nontemporal weight loads
        (1024, 256, 128, 8, 2),     # 256-row grouped tiles
    ),
)
@pytest.mark.parametrize(
    "act",
    ({"function": "relu", "limit": 4.0, "up_offset": -0.5}, {"function": "gelu", "approximate": "tanh"},
     {"function": "gelu"}, {"alpha": 1.702, "limit": 7.0, "up_offset": 1.0}),
    ids=("relu", "gelu-tanh", "gelu", "swiglu"),
)
def test_experts_bias_and_activation_every_tile_family(device, rows, hidden, intermediate, experts, topk, act):
    # Projection biases and the non-SiLU activations on each grouped kernel the chooser
    # takes; every stage against the oracle, the output against the rounding-point slack,
    # and a repeat bit for bit.
    w_gate_up, w_down = m.generate_moe_layer(hidden, intermediate, experts, 160 + rows, std=0.05)
    x = o.generate_hidden_states(rows, hidden, 161 + rows)
    ids, weights = m.generate_routes(rows, experts, topk, 162 + rows)
    generator = torch.Generator().manual_seed(163)
    act = {**act, "i_bias": torch.randn((experts, 2 * intermediate), generator=generator) * 0.5,
           "o_bias": torch.randn((experts, hidden), generator=generator) * 0.05}
    gate = GateTransform(limit=act.get("limit"), up_offset=act.get("up_offset", 0.0))
    got, operator, weights_gpu = _run_experts(device, x, w_gate_up, w_down, ids, weights, 1.25, _activation_of(act),
                                              gate, act["i_bias"], act["o_bias"])
    _check_experts(got, x, w_gate_up, w_down, ids, weights, scale=1.25, **act)
    assert_moe_stages(operator.intermediates(), x, w_gate_up, w_down, ids, weights, got, 1.25, **act)
    again = torch.empty((rows, hidden), dtype=torch.bfloat16, device=device)
    operator.run_into(hidden_states=to_device(x, device), weights=weights_gpu, topk_ids=to_device(ids, device),
                      topk_weights=to_device(weights, device), output=again)
    assert_bitwise_equal(again.cpu(), got)


def test_moe_layer_router_finalize_experts(device):
    # The reference's MoE body (registry.py:296-316): Router -> finalize -> Experts, with a
    # live-row count below the capacity.
    capacity, live, hidden, intermediate, experts, topk = 64, 40, 512, 256, 16, 4
    w_gate_up, w_down = m.generate_moe_layer(hidden, intermediate, experts, 96, std=0.05)
    generator = torch.Generator().manual_seed(97)
    projection = (torch.randn((experts, hidden), generator=generator) * 0.05).to(torch.bfloat16)
    x = o.generate_hidden_states(capacity, hidden, 98)
    x_gpu = to_device(x, device)
    router = Router(row_capacity=capacity, hidden_size=hidden, routed_expert_count=experts, routed_topk=topk,
                    device=device)
    router.run_into(hidden_states=x_gpu, router_weights=MoeRouterWeights(to_device(projection, device)))
    final_ids = torch.empty((capacity, topk), dtype=torch.int32, device=device)
    final_weights = torch.empty((capacity, topk), dtype=torch.float32, device=device)
    finalize_moe_routing(routed_ids=router.ids, routed_weights=router.weights, final_ids=final_ids,
                         final_weights=final_weights, payload_rows=torch.tensor((live,), device=device),
                         routed_expert_count=experts, shared_expert_count=0, routed_scaling_factor=1.0)
    operator = Experts(row_capacity=capacity, hidden_size=hidden, local_intermediate_size=intermediate,
                       expert_count=experts, effective_topk=topk, device=device)
    output = torch.empty_like(x_gpu)
    operator.run_into(hidden_states=x_gpu, weights=MoeFfnWeights(to_device(w_gate_up, device), to_device(w_down, device)),
                      topk_ids=final_ids, topk_weights=final_weights, output=output)
    ids, weights = m.router_topk(router.logits.cpu().float(), topk=topk, softmax=True, logits_bf16=True)
    ids, weights = m.finalize_routing(ids, weights, payload_rows=live, routed_expert_count=experts,
                                      shared_expert_count=0, routed_scaling_factor=1.0)
    assert torch.equal(final_ids.cpu(), ids)
    _check_experts(output.cpu()[:live], x[:live], w_gate_up, w_down, ids[:live], final_weights.cpu()[:live])
    assert output.cpu()[live:].abs().sum() == 0
