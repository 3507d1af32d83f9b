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
per row, weight 1 and scale 1 reduce it to ``dense_partial_reference`` bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ffn_oracle as o
from oracle import moe_oracle as m

TWO_ROWS = ((3.0, 1.0, -1.0, -3.0), (-2.0, 0.0, 2.0, 4.0))


@pytest.mark.parametrize("round_weights", (False, True))
def test_softmax_payload_router(round_weights):
    hidden = torch.tensor(TWO_ROWS, dtype=torch.bfloat16)
    logits = m.router_logits(hidden, torch.eye(4, dtype=torch.bfloat16), payload=True)
    ids, weights = m.router_topk(logits, topk=2, softmax=True, renormalize=True, round_weights=round_weights,
                                 logits_bf16=True)
    scores = torch.softmax(hidden.float(), dim=-1)
    expected_weights, expected_ids = torch.topk(scores, 2, dim=-1)
    expected_weights = expected_weights / expected_weights.sum(dim=-1, keepdim=True)
    if round_weights:
        expected_weights = expected_weights.to(torch.bfloat16).float()
    assert torch.equal(ids, expected_ids.to(torch.int32))
    assert ids.tolist() == [[0, 1], [3, 2]]
    torch.testing.assert_close(weights, expected_weights, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("corrected", (False, True))
def test_softmax_fp32_router_selection_only_correction(corrected):
    hidden = torch.tensor(TWO_ROWS, dtype=torch.bfloat16)
    bias = torch.tensor((-0.75, -0.25, 0.5, 0.8)) if corrected else None
    logits = m.router_logits(hidden, torch.eye(4, dtype=torch.bfloat16), payload=False)
    ids, weights = m.router_topk(logits, topk=2, softmax=True, correction_bias=bias, renormalize=False)
    scores = torch.softmax(hidden.float(), dim=-1)
    selection = scores if bias is None else scores + bias
    expected_ids = torch.topk(selection, 2, dim=-1).indices
    assert torch.equal(ids, expected_ids.to(torch.int32))
    torch.testing.assert_close(weights, scores.gather(1, expected_ids), rtol=1e-5, atol=1e-6)
    if corrected:
        assert not torch.equal(expected_ids, torch.topk(scores, 2, dim=-1).indices)


@pytest.mark.parametrize("experts,topk,scale", ((64, 4, 4096.0), (48, 3, None), (17, 1, 1.0), (17, 17, 1.0)))
def test_sigmoid_router_diagonal(experts, topk, scale):
    hidden = (torch.arange(2 * experts, dtype=torch.float32).view(2, experts) / (2 * experts)).to(torch.bfloat16)
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


def _reference_test_formula(x, w_gate_up, w_down, ids, weights, scale, alpha=1.0, limit=None, up_offset=0.0):
    """test_operators.py:255-281 transcribed literally (fp32 torch.mv, per route)."""

    expected = torch.zeros_like(x, dtype=torch.float32)
    for row in range(x.shape[0]):
        for slot in range(ids.shape[1]):
            expert = int(ids[row, slot])
            if expert < 0:
                continue
            projected = torch.mv(w_gate_up[expert].float(), x[row].float()).to(x.dtype)
            gate, up = projected[::2].float(), projected[1::2].float()
            if limit is not None:
                gate = gate.clamp(max=limit)
                up = up.clamp(min=-limit, max=limit)
            activated = (gate * torch.sigmoid(alpha * gate) * (up + up_offset)).to(x.dtype)
            route = torch.mv(w_down[expert].float(), activated.float())
            expected[row] += (route * weights[row, slot]).to(x.dtype).float()
        expected[row] *= scale
    return expected.to(x.dtype)


@pytest.mark.parametrize("act", ({}, {"alpha": 1.702, "limit": 7.0, "up_offset": 1.0}))
def test_experts_match_the_reference_test_formula(act):
    x, w_gate_up, w_down, ids, weights = _operator_test_case()
    got = m.experts_reference(x, w_gate_up, w_down, ids, weights, routed_scaling_factor=1.5, **act)
    expected = _reference_test_formula(x, w_gate_up, w_down, ids, weights, 1.5, **act)
    torch.testing.assert_close(got, expected, rtol=0.02, atol=0.1)
    routes = m.experts_routes(x, w_gate_up, w_down, ids, weights, **act)
    assert ((got.float() - expected.float()).abs() <= m.rounding_slack(routes, got, 1.5)).all()
    same = (got.view(torch.int16) == expected.view(torch.int16)).float().mean().item()
    assert same >= 0.95, f"only {same:.3f} of the bf16 outputs agree"
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
