"""GPU parity of the full FfnAgent path: GraphTemplates, Lanes, replays, ffn_shim.

Each case replays a template (direct kernel dispatch by default, the hipGraph where
graph dispatch is selected) and compares with the oracle's mailbox step
(gather -> RMSNorm -> Dense with the reference's rounding points -> scatter):
rows outside the gathered slots must be untouched bit-for-bit, gathered rows
meet the FFN gates of tests/parity.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from crosspool_amd import _native
from crosspool_amd.agent import FfnAgent, FfnHealthError, derive_payload_row_capacities
from crosspool_amd.ffn import DpRowLayout, ForwardMode, OutputRequirement
from crosspool_amd.ops import attach, detach, ffn_shim
from crosspool_amd.transport import FfnRequestMetadata
from crosspool_amd.weights import DenseFfnWeights
from oracle import ffn_oracle as o
from parity import assert_bitwise_equal, assert_ffn_parity, slots_tensor, to_device

from conftest import GOLDEN_DIR

pytestmark = pytest.mark.gpu


def _weights(w_gate_up, w_down, device):
    return DenseFfnWeights.from_tensors(to_device(w_gate_up, device), to_device(w_down, device))


def _check_mailbox(new_pool_gpu, pool, slots, w_gate_up, w_down, norm_weight, eps=1e-6):
    new_pool = new_pool_gpu.cpu()
    expected_pool, normalized, stage_rows = o.mailbox_step(
        pool, slots, w_gate_up, w_down, norm_weight=norm_weight, eps=eps
    )
    untouched = np.setdiff1d(np.arange(pool.shape[0]), slots)
    assert_bitwise_equal(new_pool[untouched], pool[untouched])
    fp32_rows = o.dense_fp32(normalized, w_gate_up, w_down)
    assert_ffn_parity(o.gather(new_pool, slots), stage_rows, fp32_rows)


def test_golden_mailbox_fixture(device):
    golden = np.load(GOLDEN_DIR / "mailbox_32x128.npz")
    pool = o.bf16_from_bits(golden["pool"])
    w_gate_up = o.bf16_from_bits(golden["w_gate_up"])
    w_down = o.bf16_from_bits(golden["w_down"])
    norm_weight = o.bf16_from_bits(golden["norm_weight"])
    slots = golden["slots"]
    with FfnAgent(device) as agent:
        agent.register_layer(
            instance_index=0, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device),
            norm_weight=to_device(norm_weight, device), eps=float(golden["eps"][0]),
        )
        agent.materialize(maximum_row_capacity=8)
        pool_gpu = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
        agent.lanes[0].synchronize()
        new_pool = pool_gpu.cpu()
    expected_pool = o.bf16_from_bits(golden["new_pool"])
    untouched = np.setdiff1d(np.arange(32), slots)
    assert_bitwise_equal(new_pool[untouched], expected_pool[untouched])
    normalized = o.bf16_from_bits(golden["normalized"])
    assert_ffn_parity(
        o.gather(new_pool, slots), o.bf16_from_bits(golden["ffn_rows"]), o.dense_fp32(normalized, w_gate_up, w_down)
    )


def test_config1_qwen3_0_6b_mailbox(device):
    # 256-slot mailbox, hidden 1024, 64 seeded slots, RMSNorm eps 1e-6,
    # gate_up [1024 -> 2x3072], down [3072 -> 1024], scattered back to the same slots.
    hidden, intermediate = 1024, 3072
    pool = o.generate_hidden_states(256, hidden, 17)
    w_gate_up, w_down, norm_weight = o.generate_layer(hidden, intermediate, 18)
    slots = o.generate_slots(256, 64, 19)
    with FfnAgent(device) as agent:
        agent.register_layer(
            instance_index=0, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device),
            norm_weight=to_device(norm_weight, device),
        )
        agent.materialize(maximum_row_capacity=64)
        pool_gpu = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
        agent.check_health()
    _check_mailbox(pool_gpu, pool, slots, w_gate_up, w_down, norm_weight)


@pytest.mark.parametrize("rows", [1, 4, 16, 32, 64, 256])
def test_config3_qwen3_8b_layer(device, rows):
    hidden, intermediate, pool_rows = 4096, 12288, 512
    pool = o.generate_hidden_states(pool_rows, hidden, 17)
    w_gate_up, w_down, norm_weight = o.generate_layer(hidden, intermediate, 18)
    slots = o.generate_slots(pool_rows, rows, 19)
    with FfnAgent(device) as agent:
        agent.register_layer(
            instance_index=0, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device),
            norm_weight=to_device(norm_weight, device),
        )
        agent.materialize(maximum_row_capacity=rows)
        pool_gpu = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
        agent.check_health()
    _check_mailbox(pool_gpu, pool, slots, w_gate_up, w_down, norm_weight)


@pytest.mark.parametrize("normed", [True, False])
@pytest.mark.parametrize(
    "hidden,intermediate,rows,variant",
    [
        (4096, 12288, 1, "split_gated_t8_k8_persistent+gather"),
        (4096, 12288, 8, "split_gated_t8_k8_persistent+gather"),
        (2560, 9728, 3, "split_gated_t8_k4_persistent+gather"),
        # K = 4088: the last K range ends inside a 128-wide chunk; 513 units over 512 workgroups.
        (4088, 4104, 5, "split_gated_t8_k8_persistent+gather"),
        (4096, 4096, 4, "split_gated_t8_k8_persistent+gather"),
        (1024, 3072, 1, "split_gated_t8_k4+gather"),
        (1024, 3072, 8, "split_gated_t8_k4+gather"),
        (2048, 2048, 5, "split_gated_t8_k8+gather"),
    ],
)
def test_fused_gather_matches_separate_kernels_bitwise(device, normed, hidden, intermediate, rows, variant):
    # Up to 8 rows the gather (+ RMSNorm) runs inside gate_up: the split kernel (hidden sizes
    # up to 4096) or its persistent variant (projections of at least 512 units), which stage
    # the same bits the gather kernel writes.  The kernel-level projections take the split
    # kernel with the same K ranges, so the step must equal gather kernel -> gate_up -> down
    # -> scatter bit for bit.
    from crosspool_amd import dense

    pool_rows = 256
    assert _native.dense_gate_up_variant(rows, hidden, intermediate) == variant
    pool = o.generate_hidden_states(pool_rows, hidden, 17)
    w_gate_up, w_down, norm_weight = o.generate_layer(hidden, intermediate, 18)
    slots = o.generate_slots(pool_rows, rows, 19)
    weights = _weights(w_gate_up, w_down, device)
    norm = to_device(norm_weight, device) if normed else None
    slots_d = slots_tensor(slots, device)
    with FfnAgent(device) as agent:
        agent.register_layer(instance_index=0, layer_ordinal=0, weights=weights, norm_weight=norm)
        agent.materialize(maximum_row_capacity=rows)
        pool_gpu = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_d)
        agent.check_health()
    expected = to_device(pool, device)
    x = dense.gather_rmsnorm(expected, slots_d, norm_weight=norm)
    activated = dense.gate_up_silu(x, weights.i_proj.values)
    dense.down(activated, weights.o_proj.values, out=expected, slots=slots_d)
    torch.cuda.synchronize()
    assert _native.gemm_variant(rows, 2 * intermediate, hidden, True) == (
        variant.removesuffix("+gather").removesuffix("_persistent"))
    assert_bitwise_equal(pool_gpu.cpu(), expected.cpu())
    _check_mailbox(pool_gpu, pool, slots, w_gate_up, w_down, norm_weight if normed else None)


@pytest.mark.parametrize("normed", [True, False])
@pytest.mark.parametrize(
    "hidden,intermediate,rows,gate_up,down",
    [
        (4096, 12288, 16, "resident_gated_t16_c4+gather", "stream_t16"),
        (4096, 12288, 9, "resident_gated_t16_c4+gather", "stream_t16"),
        (2560, 9728, 12, "resident_gated_t16_c3+gather", "stream_t16"),
        (2048, 6144, 16, "resident_gated_t16_c2+gather", "stream_t16"),
        (1024, 3072, 10, "resident_gated_t16_c1+gather", "split_t16_k8"),
        # K = 4088 ends inside a 128-wide chunk (a partial last chunk, padded chunks past it);
        # 2 x 4104 = 8208 gate_up rows end inside a 16-row block.
        (4088, 4104, 13, "resident_gated_t16_c4+gather", "stream_t16"),
        # the Qwen3-32B TP shard: gate_up on a separate gather (K = 5120 exceeds one part), down
        # on the resident kernel with one part
        (5120, 3200, 11, "stream_gated_t16", "resident_t16_c4"),
        # 17 to 32 rows on four token groups (gate_up of at least 16384 weight rows): the last
        # group partly live, and full
        (4096, 12288, 17, "resident_gated_t32_c4+gather", "tile_64x128_k8"),
        (4096, 12288, 32, "resident_gated_t32_c4+gather", "tile_64x128_k8"),
        (2560, 9728, 27, "resident_gated_t32_c3+gather", "tile_64x128_k8"),
        (4088, 8200, 23, "resident_gated_t32_c4+gather", "tile_64x128_k8"),
    ],
)
def test_resident_step_matches_oracle(device, normed, hidden, intermediate, rows, gate_up, down):
    # 9 to 32 rows: the token rows stay in registers of a one-per-CU grid; gate_up gathers and
    # normalises them itself (its sum of squares runs in its own order, so it agrees with the
    # gather kernel within one bf16 ulp, not bit for bit).  Checked against the oracle's
    # mailbox step; replays repeat bit for bit, also through graph dispatch.
    assert _native.dense_gate_up_variant(rows, hidden, intermediate) == gate_up
    assert _native.gemm_variant(rows, hidden, intermediate, False) == down
    pool_rows = 96
    pool = o.generate_hidden_states(pool_rows, hidden, 37)
    w_gate_up, w_down, norm_weight = o.generate_layer(hidden, intermediate, 38)
    slots = o.generate_slots(pool_rows, rows, 39)
    outputs = []
    for graph_dispatch in (False, True):
        with FfnAgent(device, graph_dispatch=graph_dispatch) as agent:
            agent.register_layer(
                instance_index=0, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device),
                norm_weight=to_device(norm_weight, device) if normed else None,
            )
            agent.materialize(maximum_row_capacity=32)
            for _ in range(2):
                pool_gpu = to_device(pool, device)
                agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
                agent.check_health()
                outputs.append(pool_gpu.cpu())
    for other in outputs[1:]:
        assert_bitwise_equal(other, outputs[0])
    _check_mailbox(outputs[0], pool, slots, w_gate_up, w_down, norm_weight if normed else None)


@pytest.mark.parametrize("hidden,intermediate,rows,gate_up", [
    (2048, 6144, 12, "resident_gated_t16_c2+gather"),
    (2048, 8192, 29, "resident_gated_t32_c2+gather"),
])
def test_resident_gather_poisons_bad_slots(device, hidden, intermediate, rows, gate_up):
    # A slot outside the mailbox: its row is staged as quiet NaNs, its output is dropped, the
    # fault bit is raised, and the other rows are their own FFN (two and four token groups;
    # with four the bad row sits in the third group).
    pool_rows = 64
    assert _native.dense_gate_up_variant(rows, hidden, intermediate) == gate_up
    pool = o.generate_hidden_states(pool_rows, hidden, 41)
    w_gate_up, w_down, norm_weight = o.generate_layer(hidden, intermediate, 42)
    slots = o.generate_slots(pool_rows, rows, 43)
    bad = slots.copy()
    bad[5 if rows <= 16 else 20] = pool_rows + 7
    with FfnAgent(device) as agent:
        agent.register_layer(
            instance_index=0, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device),
            norm_weight=to_device(norm_weight, device),
        )
        agent.materialize(maximum_row_capacity=32)
        pool_gpu = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(bad, device))
        with pytest.raises(FfnHealthError):
            agent.check_health()
    live = np.delete(slots, 5 if rows <= 16 else 20)
    _check_mailbox(pool_gpu, pool, live, w_gate_up, w_down, norm_weight)


@pytest.mark.parametrize("normed", [True, False])
@pytest.mark.parametrize("rows", [1, 6])
def test_persistent_gather_where_projections_take_the_stream_kernel(device, normed, rows):
    # Hidden 1536 (three 64-chunk groups per staged row, K ranges of three chunks): the step
    # takes the persistent gathered split kernel while the kernel-level projection takes the
    # stream kernel (other K ranges, so no bitwise comparison); checked against the oracle.
    hidden, intermediate, pool_rows = 1536, 8960, 256
    assert _native.dense_gate_up_variant(rows, hidden, intermediate) == "split_gated_t8_k4_persistent+gather"
    pool = o.generate_hidden_states(pool_rows, hidden, 27)
    w_gate_up, w_down, norm_weight = o.generate_layer(hidden, intermediate, 28)
    slots = o.generate_slots(pool_rows, rows, 29)
    with FfnAgent(device) as agent:
        agent.register_layer(
            instance_index=0, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device),
            norm_weight=to_device(norm_weight, device) if normed else None,
        )
        agent.materialize(maximum_row_capacity=8)
        pool_gpu = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
        agent.check_health()
    _check_mailbox(pool_gpu, pool, slots, w_gate_up, w_down, norm_weight if normed else None)


@pytest.mark.parametrize("rows", [3, 16])
def test_fused_gather_rows_longer_than_one_batch(device, rows):
    # Hidden 5120 is more than one load batch per lane (4096 columns), so the fused gather
    # sums the squares in batches and stages the slice in a second pass.
    hidden, intermediate, pool_rows = 5120, 3200, 64
    pool = o.generate_hidden_states(pool_rows, hidden, 27)
    w_gate_up, w_down, norm_weight = o.generate_layer(hidden, intermediate, 28)
    slots = o.generate_slots(pool_rows, rows, 29)
    with FfnAgent(device) as agent:
        agent.register_layer(
            instance_index=0,
            layer_ordinal=0,
            weights=_weights(w_gate_up, w_down, device),
            norm_weight=to_device(norm_weight, device),
        )
        agent.materialize(maximum_row_capacity=16)
        pool_gpu = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
        agent.check_health()
    _check_mailbox(pool_gpu, pool, slots, w_gate_up, w_down, norm_weight)


def test_config5_qwen3_32b_tp_shard_partial(device):
    # one of 8 TP shards, hidden 5120, shard intermediate 3200, unreduced partial.
    hidden, intermediate, rows = 5120, 3200, 8
    pool = o.generate_hidden_states(64, hidden, 17)
    w_gate_up, w_down, _ = o.generate_layer(hidden, intermediate, 18)
    slots = np.arange(rows, dtype=np.int32)
    with FfnAgent(device) as agent:
        agent.register_layer(instance_index=0, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device))
        agent.materialize(maximum_row_capacity=8)
        pool_gpu = to_device(pool, device)
        out_gpu = torch.zeros_like(pool_gpu)
        agent.execute(
            instance_index=0, layer_ordinal=0, pool=pool_gpu, out_pool=out_gpu, slots=slots_tensor(slots, device)
        )
        agent.check_health()
    assert_bitwise_equal(pool_gpu.cpu(), pool)  # the input mailbox is read-only here
    partial = out_gpu.cpu()[:rows]
    x = pool[:rows]
    assert_ffn_parity(partial, o.dense_partial_reference(x, w_gate_up, w_down), o.dense_fp32(x, w_gate_up, w_down))


def test_replay_uses_smallest_capacity_and_is_repeatable(device):
    hidden, intermediate = 1024, 3072
    pool = o.generate_hidden_states(128, hidden, 17)
    w_gate_up, w_down, norm_weight = o.generate_layer(hidden, intermediate, 18)
    slots = o.generate_slots(128, 100, 19)
    with FfnAgent(device) as agent:
        agent.register_layer(
            instance_index=0, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device),
            norm_weight=to_device(norm_weight, device),
        )
        templates = agent.materialize(maximum_row_capacity=100)
        assert sorted(t.signature.payload_row_capacity for t in templates) == [1, 2, 4, 8, 16, 32, 64, 100]
        assert agent.lanes[0].capacities(hidden, intermediate) == (1, 2, 4, 8, 16, 32, 64, 100)
        outputs = []
        for live in (5, 5, 100, 37):
            pool_gpu = to_device(pool, device)
            agent.execute(
                instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device), rows=live
            )
            agent.lanes[0].synchronize()
            outputs.append(pool_gpu.cpu())
        # Run-to-run equality of Lane outputs (test_fabric_execution.py:81).
        assert_bitwise_equal(outputs[0], outputs[1])
        for live, new_pool in zip((5, 100, 37), outputs[1:]):
            _check_mailbox(new_pool, pool, slots[:live], w_gate_up, w_down, norm_weight)
        with pytest.raises(RuntimeError, match="capacit"):
            agent.execute(instance_index=0, layer_ordinal=0, pool=to_device(pool, device),
                          slots=slots_tensor(o.generate_slots(128, 101, 3), device))


def test_layers_share_templates_and_bind_their_own_weights(device):
    # Config 2 pattern: many layers of one shape replayed through one template per capacity.
    hidden, intermediate, layers = 1024, 3072, 4
    pool = o.generate_hidden_states(4096, hidden, 17)
    slots = o.generate_slots(4096, 32, 19)
    weights = [o.generate_layer(hidden, intermediate, 100 + layer) for layer in range(layers)]
    with FfnAgent(device) as agent:
        for ordinal, (w_gate_up, w_down, norm_weight) in enumerate(weights):
            agent.register_layer(
                instance_index=0, layer_ordinal=ordinal, weights=_weights(w_gate_up, w_down, device),
                norm_weight=to_device(norm_weight, device),
            )
        templates = agent.materialize(maximum_row_capacity=256)
        assert len(templates) == 9  # capacities 1..256, shared by all four layers
        pool_gpu = to_device(pool, device)
        expected = pool
        for ordinal, (w_gate_up, w_down, norm_weight) in enumerate(weights):
            agent.execute(instance_index=0, layer_ordinal=ordinal, pool=pool_gpu, slots=slots_tensor(slots, device))
            expected, _, _ = o.mailbox_step(expected, slots, w_gate_up, w_down, norm_weight=norm_weight)
        agent.check_health()
    got = pool_gpu.cpu()
    untouched = np.setdiff1d(np.arange(4096), slots)
    assert_bitwise_equal(got[untouched], pool[untouched])
    # Four chained layers: compare with the chained stage oracle through the reference gates.
    error = o.compare(o.gather(expected, slots), o.gather(got, slots))
    assert error.normalized_rmse <= o.FFN_OUTPUT_NORMALIZED_RMSE_LIMIT


@pytest.mark.parametrize("rows", (1, 8, 32, 128, 256))
def test_config2_qwen3_0_6b_28_layer_stack(device, rows):
    # 28 independent Qwen3-0.6B FFN layers replayed through the templates of
    # one capacity set, chained on the same mailbox slots of a 4096-slot pool; every layer's
    # step is checked against the oracle fed with the GPU's own previous layer output.
    hidden, intermediate, layers = 1024, 3072, 28
    pool = o.generate_hidden_states(4096, hidden, 17)
    slots = o.generate_slots(4096, rows, 19)
    weights = [o.generate_layer(hidden, intermediate, 200 + layer) for layer in range(layers)]
    with FfnAgent(device) as agent:
        for ordinal, (w_gate_up, w_down, norm_weight) in enumerate(weights):
            agent.register_layer(
                instance_index=0, layer_ordinal=ordinal, weights=_weights(w_gate_up, w_down, device),
                norm_weight=to_device(norm_weight, device),
            )
        templates = agent.materialize(maximum_row_capacity=256)
        assert sorted(t.signature.payload_row_capacity for t in templates) == [1, 2, 4, 8, 16, 32, 64, 128, 256]
        pool_gpu = to_device(pool, device)
        slot_ids = slots_tensor(slots, device)
        previous = pool
        for ordinal, (w_gate_up, w_down, norm_weight) in enumerate(weights):
            agent.execute(instance_index=0, layer_ordinal=ordinal, pool=pool_gpu, slots=slot_ids)
            agent.lanes[0].synchronize()
            current = pool_gpu.cpu()
            _check_mailbox(current, previous, slots, w_gate_up, w_down, norm_weight)
            previous = current
        agent.check_health()


def test_layer_stack_captured_in_one_graph_matches_eager(device):
    # The replays of a layer stack captured into one hipGraph (stream capture of the direct
    # launches, as a serving step under graph capture would take them) and replayed several
    # times, with eager work and synchronisation in between: every replay equals the eager
    # stack bit for bit.
    hidden, intermediate, layers, rows = 1024, 3072, 6, 8
    pool = o.generate_hidden_states(512, hidden, 17)
    slots = slots_tensor(o.generate_slots(512, rows, 19), device)
    weights = [o.generate_layer(hidden, intermediate, 300 + layer) for layer in range(layers)]
    with FfnAgent(device) as agent:
        for ordinal, (w_gate_up, w_down, norm_weight) in enumerate(weights):
            agent.register_layer(
                instance_index=0, layer_ordinal=ordinal, weights=_weights(w_gate_up, w_down, device),
                norm_weight=to_device(norm_weight, device),
            )
        agent.materialize(maximum_row_capacity=rows)
        lane = agent.lanes[0]
        eager = to_device(pool, device)
        for ordinal in range(layers):
            lane.replay(instance_index=0, layer_ordinal=ordinal, pool=eager, slots=slots,
                        stream=torch.cuda.current_stream())
        torch.cuda.synchronize()
        graph_pool = to_device(pool, device)
        graph = torch.cuda.CUDAGraph()
        capture = torch.cuda.Stream()
        capture.wait_stream(torch.cuda.current_stream())
        with torch.cuda.graph(graph, stream=capture):
            for ordinal in range(layers):
                lane.replay(instance_index=0, layer_ordinal=ordinal, pool=graph_pool, slots=slots,
                            stream=torch.cuda.current_stream())
        for _ in range(3):
            graph_pool.copy_(to_device(pool, device))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert_bitwise_equal(graph_pool.cpu(), eager.cpu())
        agent.check_health()


def test_two_models_on_two_lanes(device):
    # Qwen3-1.7B and Qwen3-4B shaped layers share one GPU; ragged
    # per-step batches in disjoint slot ranges of an 8192-slot pool, one Lane each.
    shapes = {0: (2048, 6144), 1: (2560, 9728)}
    generator = np.random.default_rng(7)
    with FfnAgent(device, executor_lane_count=2) as agent:
        layers = {}
        for instance, (hidden, intermediate) in shapes.items():
            w_gate_up, w_down, norm_weight = o.generate_layer(hidden, intermediate, 200 + instance)
            layers[instance] = (w_gate_up, w_down, norm_weight)
            agent.register_layer(
                instance_index=instance, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device),
                norm_weight=to_device(norm_weight, device),
            )
        agent.materialize(maximum_row_capacity=512)
        pools = {i: o.generate_hidden_states(8192, h, 40 + i) for i, (h, _) in shapes.items()}
        pools_gpu = {i: to_device(p, device) for i, p in pools.items()}
        chosen = {}
        for instance in shapes:
            rows = int(generator.integers(1, 513))
            base = instance * 4096
            chosen[instance] = (base + generator.permutation(4096)[:rows]).astype(np.int32)
        for instance in shapes:
            agent.execute(
                instance_index=instance, layer_ordinal=0, pool=pools_gpu[instance],
                slots=slots_tensor(chosen[instance], device), lane=instance,
            )
        agent.check_health()
    for instance, (w_gate_up, w_down, norm_weight) in layers.items():
        _check_mailbox(pools_gpu[instance], pools[instance], chosen[instance], w_gate_up, w_down, norm_weight)


@pytest.mark.parametrize("instance", [0, 1], ids=["qwen3-1.7b", "qwen3-4b"])
def test_two_models_every_capacity_bucket(device, instance):
    # BASELINE config 4 as the bench runs it (ragged 1..512 rows per model per step, both
    # Lanes busy): every capacity bucket up to 512, at its largest and its smallest row count,
    # so each template and kernel choice the bench replays is checked against the oracle on
    # the config's own shapes.  The other model's Lane replays between the steps.
    shapes = {0: (2048, 6144), 1: (2560, 9728)}
    hidden, intermediate = shapes[instance]
    generator = np.random.default_rng(11 + instance)
    rows_list = sorted({r for c in derive_payload_row_capacities(512) for r in (c, c // 2 + 1)})
    with FfnAgent(device, executor_lane_count=2) as agent:
        layers = {}
        for index, (h, i) in shapes.items():
            w_gate_up, w_down, norm_weight = o.generate_layer(h, i, 210 + index)
            layers[index] = (w_gate_up, w_down, norm_weight)
            agent.register_layer(instance_index=index, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device),
                                 norm_weight=to_device(norm_weight, device))
        agent.materialize(maximum_row_capacity=512)
        other = 1 - instance
        other_pool = to_device(o.generate_hidden_states(1024, shapes[other][0], 50 + other), device)
        pool = o.generate_hidden_states(1024, hidden, 50 + instance)
        pool_gpu = to_device(pool, device)
        w_gate_up, w_down, norm_weight = layers[instance]
        for rows in rows_list:
            print(f"config4 instance={instance} rows={rows} gate_up={_native.dense_gate_up_variant(rows, hidden, intermediate)}",
                  flush=True)
            slots = generator.permutation(1024)[:rows].astype(np.int32)
            before = pool_gpu.cpu()
            agent.execute(instance_index=instance, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device),
                          lane=instance)
            other_slots = slots_tensor(generator.permutation(1024)[:int(generator.integers(1, 513))], device)
            agent.execute(instance_index=other, layer_ordinal=0, pool=other_pool, slots=other_slots, lane=other)
            agent.check_health()
            _check_mailbox(pool_gpu, before, slots, w_gate_up, w_down, norm_weight)


@pytest.mark.parametrize(
    "hidden,intermediate,capacity",
    # gate_up with the gather fused: the split kernel (Qwen3-0.6B), the persistent split
    # kernel (Qwen3-8B up to 8 rows) and the stream kernel (Qwen3-8B at 16 rows).
    [(1024, 3072, 4), (4096, 12288, 4), (4096, 12288, 16)],
)
def test_out_of_range_slot_sets_sticky_fault(device, hidden, intermediate, capacity):
    pool = o.generate_hidden_states(64, hidden, 17)
    w_gate_up, w_down, _ = o.generate_layer(hidden, intermediate, 18)
    with FfnAgent(device) as agent:
        agent.register_layer(instance_index=0, layer_ordinal=0, weights=_weights(w_gate_up, w_down, device))
        agent.materialize(maximum_row_capacity=capacity)
        pool_gpu = to_device(pool, device)
        # Three rows (capacity 4), or twelve for the 16-row template; slot 64 is out of range.
        live = [1, 2] if capacity <= 8 else [1, 2] + list(range(10, 20))
        bad = slots_tensor(np.array([live[0], 64, *live[1:]], dtype=np.int32), device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=bad)
        with pytest.raises(FfnHealthError):
            agent.check_health()
        assert agent.lanes[0].check_health() == _native.XP_FAULT_SLOT_OUT_OF_RANGE  # sticky
        agent.lanes[0].clear_fault()
        assert agent.lanes[0].check_health() == 0
        # A mailbox narrower than the layer's rows is refused before any kernel reads it.
        narrow = torch.zeros((64, hidden - 8), dtype=torch.bfloat16, device=device)
        with pytest.raises(ValueError, match="hidden size"):
            agent.lanes[0].replay(instance_index=0, layer_ordinal=0, pool=narrow, slots=bad)
    # The bad slot's row is staged as quiet NaNs and its output is dropped; the live rows
    # are still the FFN of their own rows and every other mailbox row is untouched.
    _check_mailbox(pool_gpu, pool, np.array(live, dtype=np.int32), w_gate_up, w_down, None)


def test_ffn_shim_matches_dense_partial(device):
    hidden, intermediate = 1024, 3072
    w_gate_up, w_down, _ = o.generate_layer(hidden, intermediate, 18)
    agent = FfnAgent(device)
    try:
        agent.register_layer(instance_index=0, layer_ordinal=3, weights=_weights(w_gate_up, w_down, device))
        agent.materialize(maximum_row_capacity=128)
        attach(agent)
        metadata = FfnRequestMetadata(3, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE, DpRowLayout.NONE)
        for rows in (1, 7, 128):
            x = o.generate_hidden_states(rows, hidden, 50 + rows)
            x_gpu = to_device(x, device)
            out = ffn_shim(x_gpu, None, metadata)
            torch.cuda.synchronize()
            assert out.shape == x.shape and out.dtype == torch.bfloat16
            assert_bitwise_equal(x_gpu.cpu(), x)
            assert_ffn_parity(
                out.cpu(), o.dense_partial_reference(x, w_gate_up, w_down), o.dense_fp32(x, w_gate_up, w_down)
            )
        with pytest.raises(RuntimeError, match="capacity"):
            ffn_shim(torch.zeros((129, hidden), dtype=torch.bfloat16, device=device), None, metadata)
        with pytest.raises(RuntimeError, match="hidden size"):
            ffn_shim(torch.zeros((4, 512), dtype=torch.bfloat16, device=device), None, metadata)
        with pytest.raises(RuntimeError, match="NONE"):
            ffn_shim(
                torch.zeros((4, hidden), dtype=torch.bfloat16, device=device),
                torch.ones(2, dtype=torch.int32, device=device),
                metadata,
            )
    finally:
        detach()
        agent.close()


@pytest.mark.parametrize(
    "hidden,intermediate,sequence",
    [
        (1024, 3072, ((0, 3), (1, 3), (0, 3), (0, 150), (1, 17), (1, 17))),
        # Qwen3-8B: the persistent split kernel (3, 8 rows), the fused stream kernel (12) and
        # the decode tiles (40), each with its dynamic LDS opt-in under capture.
        (4096, 12288, ((0, 3), (1, 3), (0, 8), (1, 12), (1, 17), (0, 40))),
    ],
)
def test_graph_dispatch_matches_direct_dispatch(device, hidden, intermediate, sequence):
    # The same replays through the instantiated hipGraphs (rebinding only changed nodes) and
    # through direct kernel launches give identical bits; alternating layers and row counts
    # exercise the rebinding.
    pool = o.generate_hidden_states(256, hidden, 17)
    layers = [o.generate_layer(hidden, intermediate, 40 + index) for index in range(2)]
    slots = slots_tensor(o.generate_slots(256, 200, 19), device)
    results = {}
    for graph_dispatch in (False, True):
        with FfnAgent(device, graph_dispatch=graph_dispatch) as agent:
            for ordinal, (w_gate_up, w_down, norm_weight) in enumerate(layers):
                agent.register_layer(
                    instance_index=0, layer_ordinal=ordinal, weights=_weights(w_gate_up, w_down, device),
                    norm_weight=to_device(norm_weight, device),
                )
            agent.materialize(maximum_row_capacity=200)
            assert agent.lanes[0].graph_dispatch is graph_dispatch
            outputs = []
            for ordinal, rows in sequence:
                pool_gpu = to_device(pool, device)
                agent.execute(instance_index=0, layer_ordinal=ordinal, pool=pool_gpu, slots=slots, rows=rows)
                agent.lanes[0].synchronize()
                outputs.append(pool_gpu.cpu())
            results[graph_dispatch] = outputs
    for direct, graph in zip(results[False], results[True]):
        assert_bitwise_equal(graph, direct)
    w_gate_up, w_down, norm_weight = layers[1]
    _check_mailbox(results[True][4], pool, slots.cpu().numpy()[:17], w_gate_up, w_down, norm_weight)
