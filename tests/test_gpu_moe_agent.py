"""GPU parity of MoE layers served by FfnAgent GraphTemplates (the MoE layer kind).

A registered MoE layer replays, from its Lane's template of the smallest capacity holding
the rows: gather (+ RMSNorm) -> Router projection and TopK -> routing finalisation (shared
experts) -> route sort -> grouped gate_up / down -> combine scattered to the slots (the
reference's captured MoE body, registry.py:242-339, on the Router-owner role).  Every stage
is checked on the GPU's own previous stage, read from the Lane workspace
(xp_moe_step_workspace_layout):

* the gathered batch within one ulp of the oracle's RMSNorm (bitwise without a norm);
* payload-dtype logits in their fp32-accumulation intervals (fp32 logits within the fp32
  sum bound);
* routed ids equal to the oracle's TopK over the GPU's logits, weights within the
  reference's rtol 1e-5 / atol 1e-6; final ids and weights equal to the oracle's finalisation;
* the Experts stages (assert_moe_stages) and the MoE output bar (assert_moe_parity) on the
  GPU's final routing;
* mailbox rows outside the slots untouched bit for bit.

Replays through the hipGraph (graph dispatch) and the standalone operator chain at the
template's capacity repeat the direct replay bit for bit.  Layers registered with fp16
weights replay with fp16 payloads and are checked at fp16 rounding points.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from crosspool_amd import _native
from crosspool_amd.agent import FfnAgent, FfnHealthError
from crosspool_amd.execution import derive_payload_row_capacities, select_capacity
from crosspool_amd.ffn import DpRowLayout, ForwardMode, GateTransform, OutputRequirement, RouterAlgorithm
from crosspool_amd.ffn import GeluActivation, ReluActivation, RouterProjectionPrecision, SiluActivation
from crosspool_amd.ffn import TopKWeightRounding
from crosspool_amd.moe import Experts, MoeFfnWeights, MoeLayerSpec, MoeRouterWeights, Router, finalize_moe_routing
from crosspool_amd.ops import attach, detach, ffn_shim
from crosspool_amd.dense import gather_rmsnorm
from crosspool_amd.transport import FfnRequestMetadata
from crosspool_amd.weights import DenseFfnWeights
from oracle import ffn_oracle as o
from oracle import moe_oracle as m
from parity import assert_bitwise_equal, assert_ffn_parity, assert_moe_parity, assert_moe_stages
from parity import assert_projection_within_bounds, assert_within_ulps, slots_tensor, to_device

pytestmark = pytest.mark.gpu


def _layer(hidden, intermediate, spec, seed, std=0.05, dtype=torch.bfloat16):
    w_gate_up, w_down = m.generate_moe_layer(hidden, intermediate, spec.expert_count, seed, std=std, dtype=dtype)
    generator = torch.Generator().manual_seed(seed + 1)
    projection = torch.randn((spec.routed_expert_count, hidden), generator=generator) * 0.05
    if spec.router_projection_precision is not RouterProjectionPrecision.FP32:
        projection = projection.to(dtype)
    correction = torch.randn((spec.routed_expert_count,), generator=generator) * 0.01
    norm_weight = (1.0 + 0.1 * torch.randn((hidden,), generator=generator)).to(dtype)
    return w_gate_up, w_down, projection, correction, norm_weight


def _act(spec, i_bias=None, o_bias=None):
    act = {}
    if isinstance(spec.activation, ReluActivation):
        act["function"] = "relu"
    elif isinstance(spec.activation, GeluActivation):
        act["function"] = "gelu"
        act["approximate"] = spec.activation.approximate
    elif spec.activation.alpha != 1.0:
        act["alpha"] = spec.activation.alpha
    if i_bias is not None:
        act["i_bias"] = i_bias
    if o_bias is not None:
        act["o_bias"] = o_bias
    if spec.gate.limit is not None:
        act["limit"] = spec.gate.limit
    if spec.gate.up_offset:
        act["up_offset"] = spec.gate.up_offset
    return act


def _lane_stages(lane, spec, hidden, intermediate, capacity, rows, dtype=torch.bfloat16):
    """The Lane workspace regions of one MoE replay at ``capacity`` (live ``rows``)."""

    desc = spec.signature(
        hidden_size=hidden, local_intermediate_size=intermediate, payload_row_capacity=capacity, payload_dtype=dtype
    ).native_descriptor()
    batch_at, logits_at, rid_at, rw_at, fid_at, fw_at, experts_at, total = _native.moe_step_workspace_layout(
        desc, capacity
    )
    workspace = lane.workspace.cpu()
    assert workspace.numel() >= total

    def view(offset, dtype, shape):
        count = int(np.prod(shape)) * dtype.itemsize
        return workspace[offset:offset + count].view(dtype).view(shape)

    fp32_logits = spec.router_projection_precision is not RouterProjectionPrecision.PAYLOAD
    routed, effective, experts = spec.routed_topk, spec.effective_topk, spec.expert_count
    offsets = (_native._SIZE * 6)()
    _native.call("xp_moe_workspace_layout", capacity, hidden, intermediate, experts, effective, offsets)
    routes = rows * effective
    return {
        "batch": view(batch_at, dtype, (rows, hidden)),
        "logits": view(logits_at, torch.float32 if fp32_logits else dtype, (rows, spec.routed_expert_count)),
        "routed_ids": view(rid_at, torch.int32, (rows, routed)),
        "routed_weights": view(rw_at, torch.float32, (rows, routed)),
        "final_ids": view(fid_at, torch.int32, (rows, effective)),
        "final_weights": view(fw_at, torch.float32, (rows, effective)),
        "experts": {
            "expert_end": view(experts_at + offsets[0], torch.int32, (experts,)),
            "sorted_route": view(experts_at + offsets[1], torch.int32, (routes,)),
            "activated": view(experts_at + offsets[4], dtype, (routes, intermediate)),
            "route_out": view(experts_at + offsets[5], dtype, (routes, hidden)),
        },
    }


def _check_replay(stages, pool, new_pool, slots, spec, w_gate_up, w_down, projection, correction, norm_weight,
                  i_bias=None, o_bias=None):
    rows = len(slots)
    dtype = pool.dtype
    untouched = np.setdiff1d(np.arange(pool.shape[0]), slots)
    assert_bitwise_equal(new_pool[untouched], pool[untouched])
    batch = stages["batch"]
    gathered = o.gather(pool, slots)
    if norm_weight is None:
        assert_bitwise_equal(batch, gathered)
    else:
        assert_within_ulps(batch, o.rmsnorm(gathered, norm_weight, 1e-6), ulps=1.0, exact_fraction=0.98)

    logits = stages["logits"]
    precision = spec.router_projection_precision
    if precision is RouterProjectionPrecision.PAYLOAD:
        # The interval is the bar; the bit-identical fraction is a sanity check that needs
        # enough logits to be meaningful (one differing logit of 72 is 1.4 %).
        assert_projection_within_bounds(logits, batch, projection, exact_fraction=0.99 if logits.numel() >= 1024 else 0.9)
    else:
        # fp32 sums of exact products (16-bit x 16-bit or widened 16-bit x fp32): the ordered-sum
        # bound K * 2^-24 * sum |x w|, doubled for the product rounding of fp32 weights.
        exact = batch.double() @ projection.double().t()
        bound = (batch.double().abs() @ projection.double().abs().t()) * (batch.shape[1] * 2.0**-23) + 1e-30
        assert bool(((logits.double() - exact).abs() <= bound).all()), "fp32 logits outside the fp32 sum bound"

    softmax = spec.router_algorithm is RouterAlgorithm.SOFTMAX
    ids, weights = m.router_topk(
        logits.float(), topk=spec.routed_topk, softmax=softmax, correction_bias=correction,
        renormalize=spec.renormalize,
        round_weights=spec.topk_weight_rounding is TopKWeightRounding.LOGITS_DTYPE,
        logits_dtype=dtype if precision is RouterProjectionPrecision.PAYLOAD else None,
    )
    assert torch.equal(stages["routed_ids"], ids)
    torch.testing.assert_close(stages["routed_weights"], weights, rtol=1e-5, atol=1e-6)
    final_ids, final_weights = m.finalize_routing(
        stages["routed_ids"], stages["routed_weights"], payload_rows=rows,
        routed_expert_count=spec.routed_expert_count, shared_expert_count=spec.shared_expert_count,
        routed_scaling_factor=spec.routed_scaling_factor,
    )
    assert torch.equal(stages["final_ids"], final_ids)
    assert torch.equal(stages["final_weights"], final_weights)

    output = o.gather(new_pool, slots)
    act = _act(spec, i_bias, o_bias)
    scale = spec.routed_scaling_factor
    assert_moe_stages(stages["experts"], batch, w_gate_up, w_down, final_ids, final_weights, output, scale, **act)
    routes = m.experts_routes(batch, w_gate_up, w_down, final_ids, final_weights, dtype=dtype, **act)
    stage = m.experts_reference(batch, w_gate_up, w_down, final_ids, final_weights, routed_scaling_factor=scale,
                                dtype=dtype, **act)
    pure = m.experts_fp32(batch, w_gate_up, w_down, final_ids, final_weights, routed_scaling_factor=scale, **act)
    assert output.dtype is dtype
    assert_moe_parity(output, stage, pure, m.rounding_slack(routes, stage, scale, dtype=dtype))


def _register(agent, spec, hidden, w_gate_up, w_down, projection, correction, norm_weight, device, ordinal=0,
              corrected=False, i_bias=None, o_bias=None):
    router = MoeRouterWeights(to_device(projection, device), to_device(correction, device) if corrected else None)
    weights = MoeFfnWeights(to_device(w_gate_up, device), to_device(w_down, device), router,
                            i_proj_bias=None if i_bias is None else to_device(i_bias, device),
                            o_proj_bias=None if o_bias is None else to_device(o_bias, device))
    agent.register_moe_layer(
        instance_index=0, layer_ordinal=ordinal, weights=weights, spec=spec,
        norm_weight=None if norm_weight is None else to_device(norm_weight, device),
    )
    return weights


# (hidden, intermediate, spec, corrected, normed, maximum capacity, replay rows)
CASES = [
    pytest.param(
        # 1 and 5 rows: gather fused into the router projection and TopK into the route sort;
        # 12 rows: TopK fused only; 33 and 64: neither.
        512, 256, MoeLayerSpec(routed_expert_count=16, routed_topk=4), False, True, 64, (1, 5, 12, 33, 64),
        id="softmax-payload-normed",
    ),
    pytest.param(
        256, 128,
        MoeLayerSpec(
            routed_expert_count=12, routed_topk=3, shared_expert_count=2, renormalize=False,
            routed_scaling_factor=2.5, router_algorithm=RouterAlgorithm.SIGMOID,
            router_projection_precision=RouterProjectionPrecision.FP32,
            activation=SiluActivation(1.702), gate=GateTransform(limit=7.0, up_offset=1.0),
        ),
        True, False, 24, (3, 17, 24),
        id="sigmoid-fp32-shared-corrected-clipped",
    ),
    pytest.param(
        512, 192,
        MoeLayerSpec(
            routed_expert_count=24, routed_topk=2, shared_expert_count=1,
            router_projection_precision=RouterProjectionPrecision.FP32_LOGITS,
            topk_weight_rounding=TopKWeightRounding.LOGITS_DTYPE, routed_scaling_factor=1.5,
        ),
        True, True, 96, (7, 96),
        id="softmax-fp32logits-shared",
    ),
    pytest.param(
        # Wide Routers: the TopK fused into the route sort (up to 16 rows) and the separate
        # TopK launch (24 rows) at 8 and 4 experts per lane.
        256, 128, MoeLayerSpec(routed_expert_count=300, routed_topk=6), False, True, 24, (2, 16, 24),
        id="softmax-300-experts",
    ),
    pytest.param(
        256, 128, MoeLayerSpec(routed_expert_count=200, routed_topk=5, router_algorithm=RouterAlgorithm.SIGMOID),
        True, False, 24, (4, 24),
        id="sigmoid-200-experts-corrected",
    ),
]


FP16_CASES = [
    pytest.param(
        512, 256, MoeLayerSpec(routed_expert_count=16, routed_topk=4), False, True, 64, (1, 5, 12, 33, 64),
        id="fp16-softmax-payload-normed",
    ),
    pytest.param(
        256, 128,
        MoeLayerSpec(
            routed_expert_count=12, routed_topk=3, shared_expert_count=2, renormalize=False,
            routed_scaling_factor=2.5, router_algorithm=RouterAlgorithm.SIGMOID,
            router_projection_precision=RouterProjectionPrecision.FP32,
            activation=SiluActivation(1.702), gate=GateTransform(limit=7.0, up_offset=1.0),
        ),
        True, False, 24, (3, 24),
        id="fp16-sigmoid-fp32-shared-corrected-clipped",
    ),
    pytest.param(
        512, 192,
        MoeLayerSpec(
            routed_expert_count=24, routed_topk=2, shared_expert_count=1,
            router_projection_precision=RouterProjectionPrecision.FP32_LOGITS,
            topk_weight_rounding=TopKWeightRounding.LOGITS_DTYPE, routed_scaling_factor=1.5,
        ),
        True, True, 96, (7, 96),
        id="fp16-softmax-fp32logits-shared",
    ),
    pytest.param(
        256, 128,
        MoeLayerSpec(routed_expert_count=200, routed_topk=5, router_algorithm=RouterAlgorithm.SIGMOID,
                     topk_weight_rounding=TopKWeightRounding.LOGITS_DTYPE),
        True, False, 24, (4, 24),
        id="fp16-sigmoid-200-experts-corrected-rounded",
    ),
]


@pytest.mark.parametrize(
    "hidden,intermediate,spec,corrected,normed,maximum,replays,dtype",
    [pytest.param(*case.values, torch.bfloat16, id=case.id) for case in CASES]
    + [pytest.param(*case.values, torch.float16, id=case.id) for case in FP16_CASES],
)
def test_moe_layer_replays_through_its_template(device, hidden, intermediate, spec, corrected, normed, maximum,
                                                replays, dtype):
    w_gate_up, w_down, projection, correction, norm_weight = _layer(hidden, intermediate, spec, 300 + hidden,
                                                                    dtype=dtype)
    if not normed:
        norm_weight = None
    pool_rows = 2 * maximum + 3
    capacities = derive_payload_row_capacities(maximum)
    with FfnAgent(device) as agent:
        _register(agent, spec, hidden, w_gate_up, w_down, projection, correction, norm_weight, device,
                  corrected=corrected)
        templates = agent.materialize(maximum_row_capacity=maximum)
        assert len(templates) == len(capacities)
        lane = agent.lanes[0]
        for rows in replays:
            print(f"case hidden={hidden} intermediate={intermediate} rows={rows} spec={spec}", flush=True)
            pool = o.generate_hidden_states(pool_rows, hidden, 400 + rows).to(dtype)
            slots = o.generate_slots(pool_rows, rows, 401 + rows)
            pool_gpu = to_device(pool, device)
            agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
            agent.check_health()
            stages = _lane_stages(lane, spec, hidden, intermediate, select_capacity(capacities, rows), rows, dtype)
            _check_replay(stages, pool, pool_gpu.cpu(), slots, spec, w_gate_up, w_down, projection,
                          correction if corrected else None, norm_weight)


@pytest.mark.parametrize("capacity,rows", ((4, 3), (16, 12), (64, 40)))
def test_moe_out_of_range_slot_sets_sticky_fault(device, capacity, rows):
    # A slot outside the mailbox: the gather (inside the Router projection at up to 8 rows,
    # its own kernel above) poisons the row and raises the Lane's sticky fault bit, and the
    # combine drops that row's output.  Every other row's result is bit for bit the one it
    # has when a valid slot takes the bad one's place (a route's output depends only on its
    # own row and expert), and mailbox rows outside the live slots stay untouched.
    hidden, intermediate, pool_rows = 512, 256, 96
    spec = MoeLayerSpec(routed_expert_count=16, routed_topk=4)
    w_gate_up, w_down, projection, correction, norm_weight = _layer(hidden, intermediate, spec, 900)
    pool = o.generate_hidden_states(pool_rows, hidden, 901)
    slots = np.asarray(o.generate_slots(pool_rows, rows, 902), dtype=np.int32)
    bad = slots.copy()
    bad[1] = pool_rows + 5
    with FfnAgent(device) as agent:
        _register(agent, spec, hidden, w_gate_up, w_down, projection, correction, norm_weight, device)
        agent.materialize(maximum_row_capacity=capacity)
        print(f"case moe bad slot capacity={capacity} rows={rows}", flush=True)
        faulty = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=faulty, slots=slots_tensor(bad, device))
        with pytest.raises(FfnHealthError):
            agent.check_health()
        assert agent.lanes[0].check_health() == _native.XP_FAULT_SLOT_OUT_OF_RANGE  # sticky
        agent.lanes[0].clear_fault()
        assert agent.lanes[0].check_health() == 0
        valid = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=valid, slots=slots_tensor(slots, device))
        agent.check_health()
        faulty, valid = faulty.cpu(), valid.cpu()
    live = np.delete(slots, 1)
    assert_bitwise_equal(faulty[live], valid[live])
    untouched = np.setdiff1d(np.arange(pool_rows), live)
    assert_bitwise_equal(faulty[untouched], pool[untouched])
    assert not torch.equal(valid[slots[1]], pool[slots[1]])  # the valid replay did write that row


@pytest.mark.parametrize(
    "spec,biases,replays",
    [
        pytest.param(  # GPT-OSS-style SwiGLU experts with both projection biases
            MoeLayerSpec(routed_expert_count=16, routed_topk=4, activation=SiluActivation(1.702),
                         gate=GateTransform(limit=7.0, up_offset=1.0)),
            3, (1, 5, 12, 33, 64), id="swiglu-both-biases",
        ),
        pytest.param(
            MoeLayerSpec(routed_expert_count=16, routed_topk=4, activation=ReluActivation(),
                         gate=GateTransform(limit=4.0, up_offset=-0.5)),
            1, (3, 40), id="relu-gate-up-bias",
        ),
        pytest.param(
            MoeLayerSpec(routed_expert_count=16, routed_topk=4, activation=GeluActivation("tanh")),
            2, (2, 64), id="gelu-tanh-down-bias",
        ),
    ],
)
def test_moe_layer_biases_and_activations_through_its_template(device, spec, biases, replays):
    # A MoE layer's projection biases (ProjectionSpec.bias_key) and the model's activation
    # go into its signature and its replays: decode sizes on the grouped split kernel, 64-row
    # grouped tiles above, every stage against the oracle.
    hidden, intermediate, maximum = 512, 256, 64
    w_gate_up, w_down, projection, correction, norm_weight = _layer(hidden, intermediate, spec, 950)
    generator = torch.Generator().manual_seed(951)
    i_bias = torch.randn((16, 2 * intermediate), generator=generator) * 0.5 if biases & 1 else None
    o_bias = torch.randn((16, hidden), generator=generator) * 0.05 if biases & 2 else None
    pool_rows = 2 * maximum + 3
    capacities = derive_payload_row_capacities(maximum)
    with FfnAgent(device) as agent:
        _register(agent, spec, hidden, w_gate_up, w_down, projection, correction, norm_weight, device,
                  i_bias=i_bias, o_bias=o_bias)
        agent.materialize(maximum_row_capacity=maximum)
        for rows in replays:
            print(f"case biases={biases} rows={rows} spec={spec}", flush=True)
            pool = o.generate_hidden_states(pool_rows, hidden, 952 + rows)
            slots = o.generate_slots(pool_rows, rows, 953 + rows)
            pool_gpu = to_device(pool, device)
            agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
            agent.check_health()
            stages = _lane_stages(agent.lanes[0], spec, hidden, intermediate, select_capacity(capacities, rows), rows)
            _check_replay(stages, pool, pool_gpu.cpu(), slots, spec, w_gate_up, w_down, projection, None,
                          norm_weight, i_bias, o_bias)


def test_moe_graph_dispatch_and_operator_chain_repeat_the_replay(device):
    hidden, intermediate, maximum = 512, 256, 64
    spec = MoeLayerSpec(routed_expert_count=16, routed_topk=4, shared_expert_count=1, routed_scaling_factor=2.0)
    w_gate_up, w_down, projection, correction, norm_weight = _layer(hidden, intermediate, spec, 500)
    pool_rows = 160
    outputs = {}
    for graph in (False, True):
        with FfnAgent(device, graph_dispatch=graph) as agent:
            _register(agent, spec, hidden, w_gate_up, w_down, projection, correction, norm_weight, device)
            agent.materialize(maximum_row_capacity=maximum)
            for rows in (3, 64, 20, 64):
                pool_gpu = to_device(o.generate_hidden_states(pool_rows, hidden, 501 + rows), device)
                slots = o.generate_slots(pool_rows, rows, 502 + rows)
                agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
                agent.check_health()
                outputs.setdefault(rows, []).append(pool_gpu.cpu())
    for rows, (direct, graphed, *again) in outputs.items():
        assert_bitwise_equal(graphed, direct)
        for repeat in again:
            assert_bitwise_equal(repeat, direct)

    # The standalone operators at the template's capacity (64 live rows): same kernels, same bits.
    rows = 64
    pool = o.generate_hidden_states(pool_rows, hidden, 501 + rows)
    slots = o.generate_slots(pool_rows, rows, 502 + rows)
    pool_gpu = to_device(pool, device)
    slots_gpu = slots_tensor(slots, device)
    batch = gather_rmsnorm(pool_gpu, slots_gpu, norm_weight=to_device(norm_weight, device), eps=1e-6)
    router = Router(row_capacity=rows, hidden_size=hidden, routed_expert_count=16, routed_topk=4, device=device)
    router_weights = MoeRouterWeights(to_device(projection, device))
    router.run_into(hidden_states=batch, router_weights=router_weights)
    final_ids = torch.empty((rows, 5), dtype=torch.int32, device=device)
    final_weights = torch.empty((rows, 5), dtype=torch.float32, device=device)
    finalize_moe_routing(routed_ids=router.ids, routed_weights=router.weights, final_ids=final_ids,
                         final_weights=final_weights, payload_rows=torch.tensor((rows,), device=device),
                         routed_expert_count=16, shared_expert_count=1, routed_scaling_factor=2.0)
    experts = Experts(row_capacity=rows, hidden_size=hidden, local_intermediate_size=intermediate, expert_count=17,
                      effective_topk=5, routed_scaling_factor=2.0, device=device)
    output = torch.empty_like(batch)
    experts.run_into(hidden_states=batch, weights=MoeFfnWeights(to_device(w_gate_up, device), to_device(w_down, device)),
                     topk_ids=final_ids, topk_weights=final_weights, output=output)
    torch.cuda.synchronize()
    assert_bitwise_equal(o.gather(outputs[rows][0], slots), output.cpu())


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16), ids=("bfloat16", "float16"))
def test_qwen3_30b_a3b_moe_layer_through_the_lane(device, dtype):
    # Qwen3-30B-A3B MoE layer: hidden 2048, moe_intermediate 768, 128 experts, top-8, softmax,
    # renormalised (norm_topk_prob), post-attention RMSNorm fused into the gather.  1 row runs
    # the gather inside the router projection and the TopK inside the route sort, 32 rows take
    # the grouped split kernel (capacity 32), 200 rows the grouped tile kernel (capacity 256).
    hidden, intermediate = 2048, 768
    spec = MoeLayerSpec(routed_expert_count=128, routed_topk=8)
    w_gate_up, w_down, projection, correction, norm_weight = _layer(hidden, intermediate, spec, 600, std=0.02,
                                                                    dtype=dtype)
    capacities = derive_payload_row_capacities(256)
    with FfnAgent(device) as agent:
        _register(agent, spec, hidden, w_gate_up, w_down, projection, correction, norm_weight, device)
        agent.materialize(maximum_row_capacity=256)
        for rows in (1, 32, 200):
            print(f"case qwen3-30b-a3b {dtype} rows={rows}", flush=True)
            pool = o.generate_hidden_states(320, hidden, 601 + rows).to(dtype)
            slots = o.generate_slots(320, rows, 602 + rows)
            pool_gpu = to_device(pool, device)
            agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
            agent.check_health()
            stages = _lane_stages(agent.lanes[0], spec, hidden, intermediate, select_capacity(capacities, rows), rows,
                                  dtype)
            _check_replay(stages, pool, pool_gpu.cpu(), slots, spec, w_gate_up, w_down, projection, None,
                          norm_weight)


def test_dense_and_moe_layers_share_one_agent_and_the_shim(device):
    # One instance mixing a Dense and a MoE layer (Qwen3-30B-A3B interleaves none, but models
    # such as DeepSeek start with Dense layers): each ordinal replays its own kind, and
    # ffn_shim serves both through the agent.
    hidden, intermediate, moe_intermediate = 512, 1024, 256
    spec = MoeLayerSpec(routed_expert_count=8, routed_topk=2)
    w_gate_up, w_down, projection, correction, _ = _layer(hidden, moe_intermediate, spec, 700)
    dense_up, dense_down, _ = o.generate_layer(hidden, intermediate, 701)
    agent = FfnAgent(device)
    try:
        agent.register_layer(
            instance_index=0, layer_ordinal=0,
            weights=DenseFfnWeights.from_tensors(to_device(dense_up, device), to_device(dense_down, device)),
        )
        _register(agent, spec, hidden, w_gate_up, w_down, projection, correction, None, device, ordinal=1)
        templates = agent.materialize(maximum_row_capacity=16)
        assert sum(t.kind == 1 for t in templates) == sum(t.kind == 2 for t in templates) == 5
        attach(agent)
        for rows in (1, 9, 16):
            x = o.generate_hidden_states(rows, hidden, 710 + rows)
            x_gpu = to_device(x, device)
            dense_meta = FfnRequestMetadata(0, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE,
                                            DpRowLayout.NONE)
            moe_meta = FfnRequestMetadata(1, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE,
                                          DpRowLayout.NONE)
            dense_out = ffn_shim(x_gpu, None, dense_meta)
            moe_out = ffn_shim(x_gpu, None, moe_meta)
            torch.cuda.synchronize()
            assert_bitwise_equal(x_gpu.cpu(), x)
            assert_ffn_parity(dense_out.cpu(), o.dense_partial_reference(x, dense_up, dense_down),
                              o.dense_fp32(x, dense_up, dense_down))
            # The shim's MoE rows against the Lane's own replay of the same rows.
            pool_gpu = x_gpu.clone()
            slots = np.arange(rows)
            agent.execute(instance_index=0, layer_ordinal=1, pool=pool_gpu, slots=slots_tensor(slots, device))
            agent.check_health()
            assert_bitwise_equal(moe_out.cpu(), pool_gpu.cpu())
            stages = _lane_stages(agent.lanes[0], spec, hidden, moe_intermediate,
                                  select_capacity(derive_payload_row_capacities(16), rows), rows)
            _check_replay(stages, x, pool_gpu.cpu(), slots, spec, w_gate_up, w_down, projection, None, None)
    finally:
        detach()
        agent.close()


def test_moe_registration_rejects_mismatched_resources(device):
    hidden, intermediate = 256, 128
    spec = MoeLayerSpec(routed_expert_count=8, routed_topk=2, shared_expert_count=1)
    w_gate_up, w_down, projection, _, _ = _layer(hidden, intermediate, spec, 800)
    with FfnAgent(device) as agent:
        no_router = MoeFfnWeights(to_device(w_gate_up, device), to_device(w_down, device))
        with pytest.raises(ValueError, match="Router projection"):
            agent.register_moe_layer(instance_index=0, layer_ordinal=0, weights=no_router, spec=spec)
        router = MoeRouterWeights(to_device(projection, device))
        short = MoeFfnWeights(to_device(w_gate_up[:8], device), to_device(w_down[:8], device), router)
        with pytest.raises(ValueError, match="experts"):
            agent.register_moe_layer(instance_index=0, layer_ordinal=0, weights=short, spec=spec)
        wide = MoeRouterWeights(to_device(projection.float(), device))
        with pytest.raises(ValueError, match="router projection"):
            agent.register_moe_layer(
                instance_index=0, layer_ordinal=0,
                weights=MoeFfnWeights(to_device(w_gate_up, device), to_device(w_down, device), wide), spec=spec,
            )
        # Payload dtypes must agree: an fp16 Router projection beside bf16 experts, an fp16
        # expert pair with a bf16 norm weight, and bf16 gate_up with fp16 down are refused.
        half_router = MoeRouterWeights(to_device(projection.half(), device))
        with pytest.raises(ValueError, match="router projection"):
            agent.register_moe_layer(
                instance_index=0, layer_ordinal=0,
                weights=MoeFfnWeights(to_device(w_gate_up, device), to_device(w_down, device), half_router),
                spec=spec,
            )
        fp16 = MoeFfnWeights(to_device(w_gate_up.half(), device), to_device(w_down.half(), device), half_router)
        with pytest.raises(ValueError, match="RMSNorm weight"):
            agent.register_moe_layer(instance_index=0, layer_ordinal=0, weights=fp16, spec=spec,
                                     norm_weight=torch.ones((hidden,), dtype=torch.bfloat16, device=device))
        with pytest.raises(ValueError, match="both"):
            MoeFfnWeights(to_device(w_gate_up, device), to_device(w_down.half(), device), router)
