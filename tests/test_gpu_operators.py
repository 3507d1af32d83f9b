"""GPU parity of the operator contract: the standalone activation, general projections
(fp16 / fp32 payloads, odd K and N, fp32 bias, fused epilogues) and the Dense operator in
CONCATENATED Gate/Up order.

Each case restates one of the reference's own operator tests (cited per test) with its
inputs and its tolerance, run through ``crosspool_amd.operators`` and, where the reference
replays, captured into a graph and replayed without allocation.  On top of the reference's
tolerance every stage is compared with the oracle (``oracle.ffn_oracle``) on the GPU's own
previous stage: within one ulp of the payload dtype (fp32: relative 1e-5), which leaves room
only for the fp32-versus-fp64 summation of the projection and the fp32 exp / erf / tanh.
"""

from __future__ import annotations

import pytest
import torch

from crosspool_amd.ffn import GateTransform, GateUpOrder, GeluActivation, ReluActivation, SiluActivation
from crosspool_amd.operators import (
    Activation,
    Dense,
    DenseExecutionPlan,
    DenseSignature,
    Gemm,
    GemmPlan,
    ProjectionLayout,
    TensorLayout,
)
from crosspool_amd.weights import DenseFfnWeights, ProjectionWeights
from oracle import ffn_oracle as o

pytestmark = pytest.mark.gpu


def ulp(values: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    mantissa = {torch.bfloat16: 7, torch.float16: 10}[dtype]
    smallest = {torch.bfloat16: -133, torch.float16: -24}[dtype]
    magnitude = values.abs().double().clamp_min(2.0**-126)
    return torch.pow(2.0, torch.maximum(torch.floor(torch.log2(magnitude)) - mantissa, torch.tensor(float(smallest))))


def assert_near_oracle(actual: torch.Tensor, expected: torch.Tensor, *, absolute: float = 0.0) -> None:
    """Within one ulp of the payload dtype (fp32: relative 1e-5), or ``absolute``, NaNs in the
    same places."""

    a = actual.detach().cpu()
    e = expected.detach().cpu().to(a.dtype)
    assert a.shape == e.shape
    nan = e.float() != e.float()
    assert torch.equal(a.float() != a.float(), nan), "NaN positions differ"
    a, e = a.double()[~nan], e.double()[~nan]
    if actual.dtype is torch.float32:
        bound = 1e-5 * e.abs() + 1e-6
    else:
        bound = ulp(e, actual.dtype)
    worst = (a - e).abs() - torch.clamp(bound, min=absolute)
    assert bool((worst <= 0).all()), f"{int((worst > 0).sum())} elements beyond one ulp (max excess {worst.max():.3e})"


def _capture(run):
    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        before = torch.cuda.memory_stats()["allocation.all.allocated"]
        run()
        after = torch.cuda.memory_stats()["allocation.all.allocated"]
    assert before == after, "capture allocated memory"
    return graph


# ------------------------------------------------------------------ standalone activation
@pytest.mark.parametrize("payload_dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("in_place", (True, False))
def test_relu_preserves_all_16bit_float_patterns(device, payload_dtype, in_place):
    # tests/suites/integration/runtime/ffnagent/test_activation.py:9-18
    values = torch.arange(65536, device=device, dtype=torch.int32).to(torch.int16).view(payload_dtype)
    expected = o.relu_bits(values.cpu()).view(torch.int16)
    output = values if in_place else torch.empty_like(values)
    Activation(function=ReluActivation(), gate=None).apply_into(inputs=values, output=output, order=None)
    torch.cuda.synchronize()
    assert torch.equal(output.view(torch.int16).cpu(), expected)


@pytest.mark.parametrize("payload_dtype,in_place", ((torch.float16, True), (torch.bfloat16, False)))
def test_ungated_silu_replays_with_caller_owned_output(device, payload_dtype, in_place):
    # test_activation.py:21-43
    inputs = torch.linspace(-12, 12, 480, device=device, dtype=payload_dtype).reshape(6, 80)
    output = inputs if in_place else torch.empty_like(inputs)
    operation = Activation(function=SiluActivation(alpha=1.3), gate=None)
    graph = _capture(lambda: operation.apply_into(inputs=inputs, output=output, order=None))
    inputs.neg_()
    reference = inputs.float().clone()
    source = inputs.clone()
    graph.replay()
    torch.cuda.synchronize()
    expected = (reference * torch.sigmoid(1.3 * reference)).to(payload_dtype)
    torch.testing.assert_close(output, expected, rtol=0.01, atol=0.01)
    assert_near_oracle(output, o.standalone_activation(source.cpu(), width=80, function="silu", gated=False,
                                                       alpha=1.3))


GATED_CASES = (
    (SiluActivation(), GateTransform(), GateUpOrder.CONCATENATED, torch.bfloat16),
    (SiluActivation(), GateTransform(), GateUpOrder.INTERLEAVED, torch.float16),
    (SiluActivation(alpha=1.702), GateTransform(limit=7.0, up_offset=1.0), GateUpOrder.CONCATENATED, torch.bfloat16),
    (SiluActivation(alpha=1.3), GateTransform(limit=4.0, up_offset=-0.5), GateUpOrder.INTERLEAVED, torch.bfloat16),
    (ReluActivation(), GateTransform(), GateUpOrder.CONCATENATED, torch.float16),
    (GeluActivation(approximate="none"), GateTransform(), GateUpOrder.CONCATENATED, torch.float16),
    (GeluActivation(approximate="tanh"), GateTransform(), GateUpOrder.INTERLEAVED, torch.bfloat16),
    (ReluActivation(), GateTransform(limit=4.0, up_offset=-0.5), GateUpOrder.INTERLEAVED, torch.bfloat16),
)


def _oracle_args(function, transform):
    name = {SiluActivation: "silu", ReluActivation: "relu", GeluActivation: "gelu"}[type(function)]
    args = dict(function=name, limit=transform.limit, up_offset=transform.up_offset)
    if isinstance(function, SiluActivation):
        args["alpha"] = function.alpha
    if isinstance(function, GeluActivation):
        args["approximate"] = function.approximate
    return args


@pytest.mark.parametrize("function,transform,order,payload_dtype", GATED_CASES)
def test_gated_activation_writes_declared_formula_and_replays_without_allocation(
    device, function, transform, order, payload_dtype
):
    # test_activation.py:46-111
    inputs = torch.linspace(-12, 12, 6 * 80, device=device, dtype=payload_dtype).reshape(6, 80)
    output = torch.empty((6, 40), device=device, dtype=payload_dtype)
    operation = Activation(function=function, gate=transform)
    graph = _capture(lambda: operation.apply_into(inputs=inputs, output=output, order=order))
    inputs.neg_()
    graph.replay()
    torch.cuda.synchronize()
    gate, up = (
        inputs.float().chunk(2, dim=-1)
        if order is GateUpOrder.CONCATENATED
        else (inputs[:, ::2].float(), inputs[:, 1::2].float())
    )
    if transform.limit is not None:
        gate = gate.clamp(max=transform.limit)
        up = up.clamp(min=-transform.limit, max=transform.limit)
    if isinstance(function, ReluActivation):
        activated = gate.relu()
    elif isinstance(function, SiluActivation):
        activated = gate * torch.sigmoid(function.alpha * gate)
    else:
        activated = torch.nn.functional.gelu(gate, approximate=function.approximate)
    expected = (activated * (up + transform.up_offset)).to(payload_dtype)
    torch.testing.assert_close(output, expected, rtol=0.01, atol=0.01)
    oracle_order = "concatenated" if order is GateUpOrder.CONCATENATED else "interleaved"
    # GELU: 1 + erf(v) cancels for v near -3.5 and below; two fp32 erf implementations differ
    # there by an fp32 ulp of 1.0, i.e. up to 0.5 |v| 2^-23 * 2 <= 1.5e-6 in the result, which can
    # exceed an fp16 ulp of the tiny values it produces.
    absolute = 2e-6 if isinstance(function, GeluActivation) else 0.0
    assert_near_oracle(output, o.standalone_activation(inputs.cpu(), width=40, gated=True, order=oracle_order,
                                                       **_oracle_args(function, transform)), absolute=absolute)


# ------------------------------------------------------------------ general projection
LINEAR_CASES = (
    (1, 2053, 66, torch.bfloat16, True),
    (17, 67, 65, torch.float16, False),
    (257, 2053, 65, torch.float32, False),
    (129, 83, 130, torch.float32, True),
    (257, 67, 65, torch.bfloat16, False),
    (256, 2048, 512, torch.bfloat16, True),
)


@pytest.mark.parametrize("rows,hidden,width,dtype,gated", LINEAR_CASES)
def test_projection_replays_current_bias_and_activation_without_allocation(device, rows, hidden, width, dtype, gated):
    # tests/suites/integration/runtime/ffnagent/test_linear.py:11-85
    generator = torch.Generator(device=device).manual_seed(101)
    projected_width = width * (2 if gated else 1)
    activation = (
        Activation(function=SiluActivation(alpha=1.3), gate=GateTransform(limit=4.0, up_offset=-0.5))
        if gated else None
    )
    layout = ProjectionLayout(
        values=TensorLayout((projected_width, hidden), dtype),
        bias=TensorLayout((projected_width,), torch.float32),
        gate_up_order=GateUpOrder.INTERLEAVED if gated else None,
    )
    plan = GemmPlan.prepare(
        input_layout=TensorLayout((rows, hidden), dtype), weight_layout=layout,
        result_layout=TensorLayout((rows, width), dtype), activation=activation,
    )
    assert plan.kernel == "projection"  # biased: the general kernel
    inputs = (torch.randn((rows, hidden), device=device, generator=generator) / hidden**0.5).to(dtype)
    projection = layout.zero_probe(device)
    projection.values.copy_(torch.randn(projection.values.shape, device=device, generator=generator) * 0.1)
    projection.bias.copy_(torch.randn(projection.bias.shape, device=device, generator=generator) * 0.1)
    output = torch.empty((rows, width), device=device, dtype=dtype)
    workspace = torch.empty(max(plan.workspace.nbytes, 16), device=device, dtype=torch.uint8)
    operation = Gemm(plan, workspace)
    graph = _capture(lambda: operation.run_into(inputs, projection, output=output))
    projection.bias.mul_(0.5)
    projection.values.mul_(0.5)
    before = torch.cuda.memory_stats()["allocation.all.allocated"]
    graph.replay()
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats()["allocation.all.allocated"] == before
    projected = torch.addmm(projection.bias.float(), inputs.float(), projection.values.float().t()).to(dtype)
    if gated:
        gate, up = projected.float()[..., ::2], projected.float()[..., 1::2]
        gate = gate.clamp_max(4.0)
        expected = (gate / (1 + torch.exp(-1.3 * gate)) * (up.clamp(-4.0, 4.0) - 0.5)).to(dtype)
    else:
        expected = projected
    torch.testing.assert_close(
        output, expected, rtol=1e-3 if dtype is torch.float32 else 0.02, atol=1e-4 if dtype is torch.float32 else 0.02
    )
    oracle = o.projection_reference(
        inputs.cpu(), projection.values.cpu(), projection.bias.cpu(),
        **(dict(function="silu", gated=True, alpha=1.3, limit=4.0, up_offset=-0.5) if gated else {}),
    )
    if gated and dtype is torch.float32:
        torch.testing.assert_close(output.cpu(), oracle, rtol=1e-5, atol=1e-6)
    elif gated:
        # the activation's input is the rounded projection, which fp32 summation may move by one
        # ulp; compare against the oracle within the reference tolerance and >= 99 % bit-identical
        torch.testing.assert_close(output.cpu(), oracle, rtol=0.02, atol=0.02)
        same = (output.cpu().view(torch.int16) == oracle.view(torch.int16)).float().mean().item()
        assert same >= 0.99, f"only {same:.4f} bit-identical to the oracle"
    else:
        assert_near_oracle(output, oracle)


def test_projection_planned_at_capacity_runs_fewer_live_rows(device):
    # The MFMA projection chooses its kernel at the live row count; Qwen3-0.6B down planned at
    # 117 rows and run at 59 takes a K split with more ranges than the plan's own choice, and
    # the plan's scratch must serve it (the largest need over 1..capacity).
    print("projection plan 117 -> live 59", flush=True)
    rows, live, hidden, width = 117, 59, 3072, 1024
    layout = ProjectionLayout(values=TensorLayout((width, hidden), torch.bfloat16))
    plan = GemmPlan.prepare(
        input_layout=TensorLayout((rows, hidden), torch.bfloat16), weight_layout=layout,
        result_layout=TensorLayout((rows, width), torch.bfloat16), activation=None,
    )
    assert plan.kernel == "down"
    generator = torch.Generator(device=device).manual_seed(117)
    inputs = torch.randn((rows, hidden), device=device, generator=generator).to(torch.bfloat16)
    projection = layout.zero_probe(device)
    projection.values.copy_(torch.randn(projection.values.shape, device=device, generator=generator) * 0.02)
    operation = Gemm(plan, torch.empty(max(plan.workspace.nbytes, 16), device=device, dtype=torch.uint8))
    for count in (live, rows, 1):
        output = torch.empty((count, width), device=device, dtype=torch.bfloat16)
        operation.run_into(inputs[:count], projection, output=output)
        torch.cuda.synchronize()
        oracle = o.projection_reference(inputs[:count].cpu(), projection.values.cpu(), None)
        torch.testing.assert_close(output.cpu(), oracle, rtol=0.02, atol=0.02)
        same = (output.cpu().view(torch.int16) == oracle.view(torch.int16)).float().mean().item()
        assert same >= 0.99, f"{count} rows: only {same:.4f} bit-identical to the oracle"


# ------------------------------------------------------------------ Dense operator
ROW_CAPACITY, HIDDEN_SIZE, LOCAL_INTERMEDIATE_SIZE = 4, 16, 8


def _dense_plan(hidden_states, layer_weights, activation):
    # tests/suites/integration/runtime/ffnagent/support.py:26-44: CONCATENATED when gated
    order = GateUpOrder.CONCATENATED if activation.gate is not None else None
    return DenseExecutionPlan.prepare(DenseSignature(
        payload_dtype=hidden_states.dtype, payload_row_capacity=hidden_states.shape[0],
        hidden_size=hidden_states.shape[1], local_intermediate_size=layer_weights.o_proj.values.shape[1],
        activation=activation, i_proj=ProjectionLayout.of(layer_weights.i_proj, order=order),
        o_proj=ProjectionLayout.of(layer_weights.o_proj),
    ))


def _check_dense_stages(operation, hidden_states, layer_weights, output, *, function, gated):
    """Each stage of the Dense operator against the oracle on the GPU's previous stage."""

    rows = hidden_states.shape[0]
    i_proj, o_proj = layer_weights.i_proj, layer_weights.o_proj
    projected = operation.projected[:rows].cpu()
    activated = operation.activated[:rows].cpu()
    bias_i = None if i_proj.bias is None else i_proj.bias.cpu()
    bias_o = None if o_proj.bias is None else o_proj.bias.cpu()
    if gated:  # CONCATENATED: plain projection, then the standalone activation
        assert_near_oracle(projected, o.projection_reference(hidden_states.cpu(), i_proj.values.cpu(), bias_i))
        assert_near_oracle(activated, o.standalone_activation(projected, width=activated.shape[1], function=function,
                                                              gated=True, order="concatenated"))
    else:  # the activation is the projection's fused epilogue
        assert_near_oracle(activated, o.projection_reference(hidden_states.cpu(), i_proj.values.cpu(), bias_i,
                                                             function=function))
    assert_near_oracle(output, o.projection_reference(activated, o_proj.values.cpu(), bias_o))


@pytest.mark.parametrize("payload_dtype", (torch.bfloat16, torch.float16), ids=("bfloat16", "float16"))
def test_dense_matches_reference_without_steady_allocation(device, payload_dtype):
    # tests/suites/integration/runtime/ffnagent/test_operators.py:25-70
    generator = torch.Generator(device=device).manual_seed(17)
    hidden_states = torch.randn((ROW_CAPACITY, HIDDEN_SIZE), device=device, generator=generator).to(payload_dtype)
    layer_weights = DenseFfnWeights(
        i_proj=ProjectionWeights(torch.randn((2 * LOCAL_INTERMEDIATE_SIZE, HIDDEN_SIZE), device=device,
                                             generator=generator).to(payload_dtype)),
        o_proj=ProjectionWeights(torch.randn((HIDDEN_SIZE, LOCAL_INTERMEDIATE_SIZE), device=device,
                                             generator=generator).to(payload_dtype)),
    )
    plan = _dense_plan(hidden_states, layer_weights, Activation(function=SiluActivation(), gate=GateTransform()))
    assert plan.i_proj.fused_activation is None  # CONCATENATED: the standalone activation runs
    workspace = torch.empty(plan.workspace.nbytes, device=device, dtype=torch.uint8)
    operation = Dense(plan, workspace)
    output = torch.empty_like(hidden_states)
    operation.run_into(hidden_states=hidden_states, layer_weights=layer_weights, output=output)
    torch.cuda.synchronize()
    allocated_before = torch.cuda.memory_allocated()
    operation.run_into(hidden_states=hidden_states, layer_weights=layer_weights, output=output)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == allocated_before
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        operation.run_into(hidden_states=hidden_states, layer_weights=layer_weights, output=output)
    hidden_states.fill_(3)
    graph.replay()
    torch.cuda.synchronize()
    gate_up = torch.mm(hidden_states.float(), layer_weights.i_proj.values.float().t()).to(payload_dtype)
    gate, up = gate_up.chunk(2, dim=-1)
    activated_up = (torch.nn.functional.silu(gate.float()) * up.float()).to(payload_dtype)
    expected = torch.mm(activated_up.float(), layer_weights.o_proj.values.float().t()).to(payload_dtype)
    torch.testing.assert_close(output, expected, rtol=0.02, atol=0.1)
    _check_dense_stages(operation, hidden_states, layer_weights, output, function="silu", gated=True)


@pytest.mark.parametrize("payload_dtype", (torch.bfloat16, torch.float16))
def test_ungated_dense_bias_and_graph_replay(device, payload_dtype):
    # test_operators.py:73-111
    generator = torch.Generator(device=device).manual_seed(19)
    hidden = torch.randn((ROW_CAPACITY, HIDDEN_SIZE), device=device, generator=generator).to(payload_dtype)
    projection = DenseFfnWeights(
        i_proj=ProjectionWeights(
            torch.randn((LOCAL_INTERMEDIATE_SIZE, HIDDEN_SIZE), device=device, generator=generator).to(payload_dtype),
            bias=torch.randn((LOCAL_INTERMEDIATE_SIZE,), device=device, generator=generator).to(payload_dtype).float(),
        ),
        o_proj=ProjectionWeights(
            torch.randn((HIDDEN_SIZE, LOCAL_INTERMEDIATE_SIZE), device=device, generator=generator).to(payload_dtype),
            bias=torch.randn((HIDDEN_SIZE,), device=device, generator=generator).to(payload_dtype).float(),
        ),
    )
    plan = _dense_plan(hidden, projection, Activation(function=ReluActivation(), gate=None))
    assert plan.i_proj.fused_activation is not None  # ungated: ReLU is the projection's epilogue
    workspace = torch.empty(plan.workspace.nbytes, device=device, dtype=torch.uint8)
    operation = Dense(plan, workspace)
    output = torch.empty_like(hidden)
    operation.run_into(hidden_states=hidden, layer_weights=projection, output=output)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        operation.run_into(hidden_states=hidden, layer_weights=projection, output=output)
    hidden.mul_(0.5)
    graph.replay()
    torch.cuda.synchronize()
    first, second = projection.i_proj, projection.o_proj
    activated = torch.addmm(first.bias.to(payload_dtype).float(), hidden.float(), first.values.float().t()).to(
        payload_dtype).relu()
    expected = torch.addmm(second.bias.to(payload_dtype).float(), activated.float(), second.values.float().t()).to(
        payload_dtype)
    torch.testing.assert_close(output, expected, rtol=0.02, atol=0.1)
    _check_dense_stages(operation, hidden, projection, output, function="relu", gated=False)


def test_dense_projection_bias_preserves_fused_rounding_without_capture_allocation(device):
    # tests/suites/integration/runtime/ffnagent/test_projection.py:86-139
    generator = torch.Generator(device=device).manual_seed(37)
    layer = DenseFfnWeights(
        i_proj=ProjectionWeights(torch.randn((16, 16), device=device, generator=generator).to(torch.bfloat16),
                                 bias=torch.linspace(-2, 2, 16, dtype=torch.bfloat16, device=device).float()),
        o_proj=ProjectionWeights(torch.randn((16, 8), device=device, generator=generator).to(torch.bfloat16),
                                 bias=torch.linspace(-2, 2, 16, dtype=torch.bfloat16, device=device).float()),
    )
    hidden = torch.randn((4, 16), dtype=torch.bfloat16, device=device, generator=generator)
    output = torch.empty_like(hidden)
    plan = _dense_plan(hidden, layer, Activation(function=SiluActivation(), gate=GateTransform()))
    workspace = torch.empty(plan.workspace.nbytes, device=device, dtype=torch.uint8)
    operation = Dense(plan, workspace)
    graph = _capture(lambda: operation.run_into(hidden_states=hidden, layer_weights=layer, output=output))
    hidden.mul_(0.5)
    graph.replay()
    torch.cuda.synchronize()
    projected = (hidden.float() @ layer.i_proj.values.float().t() + layer.i_proj.bias.float()).to(hidden.dtype)
    gate, up = projected.float().chunk(2, dim=-1)
    activated = (gate * torch.sigmoid(gate) * up).to(hidden.dtype)
    expected = (activated.float() @ layer.o_proj.values.float().t() + layer.o_proj.bias.float()).to(hidden.dtype)
    torch.testing.assert_close(output, expected, rtol=0.02, atol=0.1)
    _check_dense_stages(operation, hidden, layer, output, function="silu", gated=True)
