"""CPU pins of the MoE oracle (oracle/moe_oracle.py).

Known answers come from the reference's own routing and operator tests (paths relative to
the CrossPool checkout):

* tests/suites/integration/runtime/ffnagent/routing/test_softmax_payload.py:17-56;
* routing/test_softmax_fp32.py:17-67 (selection-only correction changes the picks);
* routing/test_sigmoid.py:14-73 (diagonal projections) and :76-117 (tie policy);
* routing/test_metadata.py:8-80 (finalisation, including the dynamic live-row count);
* test_operators.py:121-281 (the Experts expected-value formula, here transcribed a second
  time in fp32 with torch.mv exactly as the test writes it).

The Experts oracle is also tied to the already-pinned Dense oracle: one expert, one route
per row, weight 1 and scale 1 reduce it to ``dense_partial_reference`` bit for bit.  The
router and Experts pins run with bf16 and fp16 payloads, as the reference's tests are
parametrized; the fp16 rounding points are pinned further by an exact-rational brute force
with its own binary16 rounding rule.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import ffn_oracle as o
from oracle import moe_oracle as m

TWO_ROWS = ((3.0, 1.0, -1.0, -3.0), (-2.0, 0.0, 2.0, 4.0))
PAYLOADS = pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16), ids=("bfloat16", "float16"))


@PAYLOADS
@pytest.mark.parametrize("round_weights", (False, True))
def test_softmax_payload_router(round_weights, dtype):
    hidden = torch.tensor(TWO_ROWS, dtype=dtype)
    logits = m.router_logits(hidden, torch.eye(4, dtype=dtype), payload=True, dtype=dtype)
    ids, weights = m.router_topk(logits, topk=2, softmax=True, renormalize=True, round_weights=round_weights,
                                 logits_dtype=dtype)
    scores = torch.softmax(hidden.float(), dim=-1)
    expected_weights, expected_ids = torch.topk(scores, 2, dim=-1)
    expected_weights = expected_weights / expected_weights.sum(dim=-1, keepdim=True)
    unrounded = expected_weights
    if round_weights:
        # The reference takes the LOGITS_DTYPE weights from a TopK over the payload-dtype
        # logits, whose values are in that dtype.
        expected_weights = expected_weights.to(dtype).float()
    assert torch.equal(ids, expected_ids.to(torch.int32))
    assert ids.tolist() == [[0, 1], [3, 2]]
    torch.testing.assert_close(weights, expected_weights, rtol=1e-5, atol=1e-6)
    if round_weights:
        # The other 16-bit rounding is far outside the tolerance: the dtype is pinned.
        other = torch.float16 if dtype is torch.bfloat16 else torch.bfloat16
        assert not torch.allclose(weights, unrounded.to(other).float(), rtol=1e-5, atol=1e-6)


@PAYLOADS
@pytest.mark.parametrize("corrected", (False, True))
def test_softmax_fp32_router_selection_only_correction(corrected, dtype):
    hidden = torch.tensor(TWO_ROWS, dtype=dtype)
    bias = torch.tensor((-0.75, -0.25, 0.5, 0.8)) if corrected else None
    logits = m.router_logits(hidden, torch.eye(4, dtype=dtype), payload=False)
    ids, weights = m.router_topk(logits, topk=2, softmax=True, correction_bias=bias, renormalize=False)
    scores = torch.softmax(hidden.float(), dim=-1)
    selection = scores if bias is None else scores + bias
    expected_ids = torch.topk(selection, 2, dim=-1).indices
    assert torch.equal(ids, expected_ids.to(torch.int32))
    torch.testing.assert_close(weights, scores.gather(1, expected_ids), rtol=1e-5, atol=1e-6)
    if corrected:
        assert not torch.equal(expected_ids, torch.topk(scores, 2, dim=-1).indices)


@PAYLOADS
@pytest.mark.parametrize("experts,topk,scale", ((64, 4, 4096.0), (48, 3, None), (17, 1, 1.0), (17, 17, 1.0)))
def test_sigmoid_router_diagonal(experts, topk, scale, dtype):
    hidden = torch.arange(2 * experts, dtype=torch.float32).view(2, experts).to(dtype) / (2 * experts)
    bias = torch.linspace(-0.25, 0.25, experts) * scale if scale is not None else None
    projection = torch.diag(torch.linspace(0.101, 1.909, experts))
    logits = m.router_logits(hidden, projection, payload=False)
    ids, weights = m.router_topk(logits, topk=topk, softmax=False, correction_bias=bias, renormalize=True)
    scores = torch.sigmoid(hidden.float() @ projection.t())
    selection = scores if bias is None else scores + bias
    expected_ids = torch.topk(selection, topk, dim=-1).indices
    expected_weights = torch.gather(scores, 1, expected_ids)
    expected_weights = expected_weights / expected_weights.sum(dim=-1, keepdim=True)
    order, expected_order = ids.argsort(dim=-1), expected_ids.argsort(dim=-1)
    assert torch.equal(ids.gather(1, order), expected_ids.gather(1, expected_order).to(torch.int32))
    torch.testing.assert_close(weights.gather(1, order), expected_weights.gather(1, expected_order), rtol=1e-5,
                               atol=1e-6)


@pytest.mark.parametrize("softmax", (True, False))
def test_router_tie_policy(softmax):
    # routing/test_sigmoid.py:76-117: ties go to low ids for softmax, high ids for sigmoid,
    # and zero sigmoid scores keep zero weights after renormalisation.
    hidden = torch.tensor(((0.0,) * 17, (-1000.0,) * 17), dtype=torch.bfloat16)
    logits = m.router_logits(hidden, torch.eye(17, dtype=torch.bfloat16), payload=softmax)
    ids, weights = m.router_topk(logits, topk=3, softmax=softmax, renormalize=True, logits_bf16=softmax)
    expected_ids = (0, 1, 2) if softmax else (16, 15, 14)
    second = (1 / 3, 1 / 3, 1 / 3) if softmax else (0.0, 0.0, 0.0)
    assert ids.tolist() == [list(expected_ids)] * 2
    torch.testing.assert_close(weights, torch.tensor(((1 / 3, 1 / 3, 1 / 3), second)), rtol=1e-5, atol=1e-6)


def test_finalize_routing_known_answers():
    # routing/test_metadata.py:8-80
    routed_ids = torch.tensor(((0, 2), (1, 3), (2, 0), (3, 1)), dtype=torch.int32)
    routed_weights = torch.tensor(((0.75, 0.25), (0.6, 0.4), (0.9, 0.1), (0.55, 0.45)))
    kwargs = dict(routed_expert_count=4, shared_expert_count=1, routed_scaling_factor=2.0)
    ids, weights = m.finalize_routing(routed_ids, routed_weights, payload_rows=2, **kwargs)
    assert ids.tolist() == [[0, 2, 4], [1, 3, 4], [-1, -1, -1], [-1, -1, -1]]
    expected = torch.tensor(((0.75, 0.25, 0.5), (0.6, 0.4, 0.5), (0.0,) * 3, (0.0,) * 3))
    torch.testing.assert_close(weights, expected, rtol=0, atol=0)
    ids, weights = m.finalize_routing(routed_ids, routed_weights, payload_rows=3, **kwargs)
    assert ids[2].tolist() == [2, 0, 4] and ids[3].tolist() == [-1, -1, -1]
    torch.testing.assert_close(weights[2], torch.tensor((0.9, 0.1, 0.5)), rtol=0, atol=0)
    ids, weights = m.finalize_routing(torch.zeros_like(routed_ids), torch.zeros_like(routed_weights),
                                      payload_rows=3, **kwargs)
    assert weights[:3, :2].abs().sum() == 0 and weights[:3, 2].tolist() == [0.5] * 3


def _operator_test_case(payload_dtype=torch.bfloat16):
    # test_operators.py:133-165: four experts, two slots, a dead row.
    generator = torch.Generator().manual_seed(31)
    x = (torch.randn((4, 16), generator=generator) / 4).to(payload_dtype)
    w_gate_up = (torch.randn((4, 16, 16), generator=generator) / 4).to(payload_dtype)
    w_down = (torch.randn((4, 16, 8), generator=generator) / 4).to(payload_dtype)
    ids = torch.tensor(((0, 1), (2, 3), (1, 3), (-1, -1)), dtype=torch.int32)
    weights = torch.tensor(((0.75, 0.25), (0.6, 0.4), (0.9, 0.1), (0.0, 0.0)))
    return x, w_gate_up, w_down, ids, weights


def _reference_test_formula(x, w_gate_up, w_down, ids, weights, scale, alpha=1.0, limit=None, up_offset=0.0,
                            function="silu", approximate="none", i_bias=None, o_bias=None):
    """test_operators.py:255-281 transcribed literally (fp32 torch.mv, per route; torch's own
    relu / gelu for the other activations)."""

    expected = torch.zeros_like(x, dtype=torch.float32)
    for row in range(x.shape[0]):
        for slot in range(ids.shape[1]):
            expert = int(ids[row, slot])
            if expert < 0:
                continue
            projected = torch.mv(w_gate_up[expert].float(), x[row].float())
            if i_bias is not None:
                projected += i_bias[expert]
            projected = projected.to(x.dtype)
            gate, up = projected[::2].float(), projected[1::2].float()
            if limit is not None:
                gate = gate.clamp(max=limit)
                up = up.clamp(min=-limit, max=limit)
            if function == "relu":
                activated = gate.relu()
            elif function == "gelu":
                activated = torch.nn.functional.gelu(gate, approximate=approximate)
            else:
                activated = gate * torch.sigmoid(alpha * gate)
            activated = (activated * (up + up_offset)).to(x.dtype)
            route = torch.mv(w_down[expert].float(), activated.float())
            if o_bias is not None:
                route += o_bias[expert]
            expected[row] += (route * weights[row, slot]).to(x.dtype).float()
        expected[row] *= scale
    return expected.to(x.dtype)


# test_operators.py:110-121: payload dtype, projection biases, activation and gate transform.
OPERATOR_CASES = [
    pytest.param(torch.bfloat16, False, {}, id="bf16-silu"),
    pytest.param(torch.float16, False, {}, id="fp16-silu"),
    pytest.param(torch.bfloat16, True, {}, id="bf16-bias-silu"),
    pytest.param(torch.bfloat16, True, {"alpha": 1.702, "limit": 7.0, "up_offset": 1.0}, id="bf16-bias-swiglu"),
    pytest.param(torch.bfloat16, True, {"function": "relu", "limit": 4.0, "up_offset": -0.5}, id="bf16-bias-relu"),
    pytest.param(torch.bfloat16, True, {"function": "gelu"}, id="bf16-bias-gelu"),
    pytest.param(torch.bfloat16, True, {"function": "gelu", "approximate": "tanh"}, id="bf16-bias-gelu-tanh"),
]


def _operator_biases(with_bias: bool):
    # test_operators.py:216-226: randn fp32 biases of i_proj [E, 2I] and o_proj [E, H].
    if not with_bias:
        return {}
    generator = torch.Generator().manual_seed(32)
    return {"i_bias": torch.randn((4, 16), generator=generator), "o_bias": torch.randn((4, 16), generator=generator)}


@pytest.mark.parametrize("dtype,with_bias,act", OPERATOR_CASES)
def test_experts_match_the_reference_test_formula(dtype, with_bias, act):
    # Every parametrization of test_operators.py:110-121.
    x, w_gate_up, w_down, ids, weights = _operator_test_case(dtype)
    act = {**act, **_operator_biases(with_bias)}
    got = m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5, dtype=dtype, **act)
    assert got.dtype is dtype
    expected = _reference_test_formula(x, w_gate_up, w_down, ids, weights, 1.5, **act)
    torch.testing.assert_close(got, expected, rtol=0.02, atol=0.1)
    routes = m.experts_routes(x, w_gate_up, w_down, ids, weights, dtype=dtype, **act)
    assert ((got.float() - expected.float()).abs() <= m.rounding_slack(routes, got, 1.5, dtype=dtype)).all()
    same = (got.view(torch.int16) == expected.view(torch.int16)).float().mean().item()
    assert same >= 0.95, f"only {same:.3f} of the outputs agree"
    assert got[3].abs().sum() == 0  # the dead row
    pure = m.experts_fp32(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5, **act)
    assert o.compare(pure, got.float()).rel_l2 < 1e-2


def test_experts_reduce_to_the_dense_oracle():
    hidden, intermediate = 64, 32
    w_gate_up, w_down, _ = o.generate_layer(hidden, intermediate, 5, std=0.2)
    x = o.generate_hidden_states(9, hidden, 6)
    ids = torch.zeros((9, 1), dtype=torch.int32)
    weights = torch.ones((9, 1))
    got = m.experts_reference(x, w_gate_up.unsqueeze(0), w_down.unsqueeze(0), ids, weights)
    assert torch.equal(got.view(torch.int16), o.dense_partial_reference(x, w_gate_up, w_down).view(torch.int16))


def test_experts_invariants_and_planted_mistakes():
    x, w_gate_up, w_down, ids, weights = _operator_test_case()
    base = m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5)
    assert m.experts_reference(x, w_gate_up, w_down, ids, torch.zeros_like(weights)).abs().sum() == 0
    # Swapping a row's two slots changes only the fp32 summation order.
    swapped = m.experts_reference(x, w_gate_up, w_down, ids.flip(1), weights.flip(1), routed_scaling_factor=1.5)
    assert (swapped.float() - base.float()).abs().max() <= o.bf16_ulp(base.float()).max()
    expected = _reference_test_formula(x, w_gate_up, w_down, ids, weights, 1.5)
    # Planted mistakes (Gate/Up swapped, the route weight dropped, the scale dropped) all
    # move the output by more than 5 % rel-L2; the correct oracle stays within 1 %.
    assert o.compare(expected.float(), base.float()).rel_l2 < 0.01
    gate_up_swapped = w_gate_up.view(4, 8, 2, 16).flip(2).reshape(4, 16, 16)
    for wrong in (
        m.experts_reference(x, gate_up_swapped, w_down, ids, weights, routed_scaling_factor=1.5),
        m.experts_reference(x, w_gate_up, w_down, ids, torch.ones_like(weights), routed_scaling_factor=1.5),
        m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.0),
    ):
        assert o.compare(expected.float(), wrong.float()).rel_l2 > 0.05


def _f16(value: float) -> float:
    """Round-to-nearest-even to IEEE binary16 (11 significant bits, subnormal spacing 2^-24),
    computed on exact rationals (independent of torch's conversion)."""

    if value == 0:
        return value
    _, exponent = math.frexp(value)  # 2^(exponent-1) <= |value| < 2^exponent
    quantum = Fraction(2) ** max(exponent - 11, -24)
    scaled = Fraction(value) / quantum
    floor = math.floor(scaled)
    remainder = scaled - floor
    if remainder > Fraction(1, 2) or (remainder == Fraction(1, 2) and floor % 2 == 1):
        floor += 1
    return float(floor * quantum)


def test_fp16_experts_match_exact_brute_force():
    # The reference's operator case (test_operators.py:114, fp16 payload) by exact rationals:
    # projections rounded through fp32 to binary16, fp32 SiLU*up rounded to binary16, exact
    # down projection times the route weight in fp32 rounded to binary16, fp32 sum over the
    # slots in order times the scale rounded to binary16.  A bf16 rounding point left in the
    # oracle (8 significant bits instead of 11) fails here.
    x, w_gate_up, w_down, ids, weights = _operator_test_case(torch.float16)

    def exact(row, matrix):
        return [sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(row, w_row)) for w_row in matrix]

    expected = []
    for row in range(4):
        columns = [np.float32(0)] * x.shape[1]
        for slot in range(2):
            expert = int(ids[row, slot])
            if expert < 0:
                continue
            projected = [_f16(float(np.float32(float(v)))) for v in exact(x[row].tolist(), w_gate_up[expert].tolist())]
            activated = []
            for gate, up in zip(projected[0::2], projected[1::2]):
                g = np.float32(gate)
                silu = np.float32(g / (np.float32(1) + np.exp(-g, dtype=np.float32)))
                activated.append(_f16(float(np.float32(silu * np.float32(up)))))
            gamma = np.float32(float(weights[row, slot]))
            routes = [_f16(float(np.float32(np.float32(float(r)) * gamma)))
                      for r in exact(activated, w_down[expert].tolist())]
            columns = [np.float32(c + np.float32(r)) for c, r in zip(columns, routes)]
        expected.append([_f16(float(np.float32(c * np.float32(1.5)))) for c in columns])
    got = m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5, dtype=torch.float16)
    assert got.dtype is torch.float16
    assert got.float().tolist() == expected
    # The bf16 oracle on the same values is a different function.
    bf16 = m.experts_reference(x.bfloat16(), w_gate_up.bfloat16(), w_down.bfloat16(), ids, weights,
                               routed_scaling_factor=1.5)
    assert not torch.equal(got.float(), bf16.float())


def test_fp16_router_logits_round_to_binary16():
    x, w_gate_up, _, _, _ = _operator_test_case(torch.float16)
    projection = w_gate_up[0, :6]
    logits = m.router_logits(x, projection, payload=True, dtype=torch.float16)
    brute = [[_f16(float(np.float32(float(sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(row, w))))))
              for w in projection.tolist()] for row in x.tolist()]
    assert logits.tolist() == brute
    # fp16 sigmoid selection: rounding the selection to binary16 can merge two scores that
    # fp32 keeps apart; the tie then goes to the higher id.
    scores = torch.tensor(((0.0, 0.0),))
    bias = torch.tensor((2.0**-11, 0.0))
    ids, _ = m.router_topk(scores, topk=1, softmax=False, correction_bias=bias, logits_dtype=torch.float16)
    assert ids.tolist() == [[0]]  # 0.5 + 2^-11 is representable in binary16 (spacing 2^-11 at 0.5)
    bias = torch.tensor((2.0**-12, 0.0))
    ids, _ = m.router_topk(scores, topk=1, softmax=False, correction_bias=bias, logits_dtype=torch.float16)
    assert ids.tolist() == [[1]]  # 0.5 + 2^-12 rounds to 0.5 (ties to even): a tie, won by the higher id
    ids, _ = m.router_topk(scores, topk=1, softmax=False, correction_bias=bias)
    assert ids.tolist() == [[0]]  # in fp32 the two stay apart
    bias = torch.tensor((2.0**-9, 0.0))
    ids, _ = m.router_topk(scores, topk=1, softmax=False, correction_bias=bias, logits_dtype=torch.bfloat16)
    assert ids.tolist() == [[1]]  # bf16 (spacing 2^-8 at 0.5) merges what binary16 keeps apart
    ids, _ = m.router_topk(scores, topk=1, softmax=False, correction_bias=bias, logits_dtype=torch.float16)
    assert ids.tolist() == [[0]]


def test_experts_bias_and_activation_planted_mistakes():
    # With the reference's biased cases, dropping either bias, or evaluating another
    # activation, moves the output by more than 5 % rel-L2 from the reference's formula;
    # the oracle stays within 1 %.
    x, w_gate_up, w_down, ids, weights = _operator_test_case()
    biases = _operator_biases(True)
    for act in ({"function": "relu", "limit": 4.0, "up_offset": -0.5}, {"function": "gelu"}, {}):
        expected = _reference_test_formula(x, w_gate_up, w_down, ids, weights, 1.5, **act, **biases).float()
        good = m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5, **act, **biases)
        assert o.compare(expected, good.float()).rel_l2 < 0.01
        other = {"function": "silu"} if act.get("function") else {"function": "gelu"}
        for wrong in (
            m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5, **act,
                                o_bias=biases["o_bias"]),
            m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5, **act,
                                i_bias=biases["i_bias"]),
            m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5,
                                **{**act, **other}, **biases),
        ):
            assert o.compare(expected, wrong.float()).rel_l2 > 0.05
