"""fp16 payloads through the FfnAgent path.

The reference admits bf16 and fp16 payloads (is_supported_payload_dtype,
src/cext-include/xpool/ffn.hpp:83-85): the shim checks the caller's tensor against the
arena's payload dtype (src/cext/transport/instance.cpp:104-105) and the loader keeps an
fp16 checkpoint in fp16 (loader.py:485-508).  Here every Dense kernel is instantiated for
fp16 as well (v_mfma_f32_16x16x32_f16 / 32x32x16_f16, fp16 rounding points in the
epilogues and the fused RMSNorm), and a layer registered with fp16 weights is replayed
from fp16 templates.  Each case is checked against the oracle with fp16 rounding points
(o.mailbox_step rounds the norm, gate/up, the activation and the output to the payload
dtype) under the FFN parity gates of tests/parity.py, at every kernel family the chooser
takes: the split kernel with the gather fused and its persistent variant, the resident
kernel, the decode tiles and the MFMA-bound tiles.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from crosspool_amd import _native
from crosspool_amd.agent import FfnAgent, FfnHealthError
from crosspool_amd.ffn import DpRowLayout, ForwardMode, OutputRequirement
from crosspool_amd.ops import attach, detach, ffn_shim
from crosspool_amd.transport import FfnRequestMetadata
from crosspool_amd.weights import DenseFfnWeights
from oracle import ffn_oracle as o
from parity import assert_bitwise_equal, assert_ffn_parity, slots_tensor, to_device

pytestmark = pytest.mark.gpu

DECODE = FfnRequestMetadata(0, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE, DpRowLayout.NONE)
F16_NAN = 0x7E00


def _fp16_layer(hidden: int, intermediate: int, seed: int):
    """N(0, 0.02) weights and a 1 + N(0, 0.1) norm weight drawn in fp32, stored in fp16."""

    generator = torch.Generator().manual_seed(seed)
    w_gate_up = (torch.randn((2 * intermediate, hidden), generator=generator) * 0.02).half()
    w_down = (torch.randn((hidden, intermediate), generator=generator) * 0.02).half()
    norm_weight = (1 + 0.1 * torch.randn((hidden,), generator=generator)).half()
    return w_gate_up.contiguous(), w_down.contiguous(), norm_weight.contiguous()


def _check(new_pool_gpu, pool, slots, w_gate_up, w_down, norm_weight):
    new_pool = new_pool_gpu.cpu()
    assert new_pool.dtype is torch.float16
    _, normalized, stage_rows = o.mailbox_step(pool, slots, w_gate_up, w_down, norm_weight=norm_weight)
    assert stage_rows.dtype is torch.float16
    untouched = np.setdiff1d(np.arange(pool.shape[0]), slots)
    assert_bitwise_equal(new_pool[untouched], pool[untouched])
    assert_ffn_parity(o.gather(new_pool, slots), stage_rows, o.dense_fp32(normalized, w_gate_up, w_down))


@pytest.mark.parametrize(
    "hidden,intermediate,rows,gate_up",
    [
        (1024, 3072, 3, "split_gated_t8_k4+gather"),
        (1024, 3072, 12, "resident_gated_t16_c1+gather"),
        (1024, 3072, 40, "tile_gated_64x64"),
        (1024, 3072, 300, "tile_gated_64x128"),
        (4096, 12288, 1, "split_gated_t8_k8_persistent+gather"),
        (4096, 12288, 16, "resident_gated_t16_c4+gather"),
        (4096, 12288, 32, "resident_gated_t32_c4+gather"),
        (4096, 12288, 2048, "tile_gated_256x256"),
    ],
)
def test_fp16_layer_matches_oracle(device, hidden, intermediate, rows, gate_up):
    print(f"fp16 layer {hidden}x{intermediate} rows={rows}", flush=True)
    assert _native.dense_gate_up_variant(rows, hidden, intermediate) == gate_up
    pool_rows = max(2 * rows, 64)
    pool = o.generate_hidden_states(pool_rows, hidden, 61).half()
    w_gate_up, w_down, norm_weight = _fp16_layer(hidden, intermediate, 62)
    slots = o.generate_slots(pool_rows, rows, 63)
    weights = DenseFfnWeights.from_tensors(to_device(w_gate_up, device), to_device(w_down, device))
    with FfnAgent(device) as agent:
        agent.register_layer(
            instance_index=0, layer_ordinal=0, weights=weights, norm_weight=to_device(norm_weight, device)
        )
        agent.materialize(maximum_row_capacity=rows)
        assert agent.lanes[0].capacities(hidden, intermediate, torch.float16)[-1] == rows
        assert agent.lanes[0].capacities(hidden, intermediate, torch.bfloat16) == ()
        pool_gpu = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
        agent.check_health()
        # A bf16 mailbox is refused for an fp16 layer before any kernel reads it.
        with pytest.raises(ValueError, match="payload dtype"):
            agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu.bfloat16(),
                          slots=slots_tensor(slots, device))
    _check(pool_gpu, pool, slots, w_gate_up, w_down, norm_weight)


def test_bf16_and_fp16_layers_share_an_agent(device):
    # One agent, one Lane: a bf16 and an fp16 layer of one shape get templates of their own
    # payload dtype; replays alternate between them.
    hidden, intermediate, rows, pool_rows = 2048, 6144, 24, 96
    w_gate_up16, w_down16, norm16 = _fp16_layer(hidden, intermediate, 71)
    w_gate_up, w_down, norm = o.generate_layer(hidden, intermediate, 72)
    slots = o.generate_slots(pool_rows, rows, 73)
    pool16 = o.generate_hidden_states(pool_rows, hidden, 74).half()
    pool = o.generate_hidden_states(pool_rows, hidden, 75)
    with FfnAgent(device) as agent:
        agent.register_layer(instance_index=0, layer_ordinal=0, norm_weight=to_device(norm16, device),
                             weights=DenseFfnWeights.from_tensors(to_device(w_gate_up16, device),
                                                                  to_device(w_down16, device)))
        agent.register_layer(instance_index=0, layer_ordinal=1, norm_weight=to_device(norm, device),
                             weights=DenseFfnWeights.from_tensors(to_device(w_gate_up, device),
                                                                  to_device(w_down, device)))
        agent.materialize(maximum_row_capacity=32)
        pool16_gpu, pool_gpu = to_device(pool16, device), to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool16_gpu, slots=slots_tensor(slots, device))
        agent.execute(instance_index=0, layer_ordinal=1, pool=pool_gpu, slots=slots_tensor(slots, device))
        agent.check_health()
    _check(pool16_gpu, pool16, slots, w_gate_up16, w_down16, norm16)
    new_pool = pool_gpu.cpu()
    _, normalized, stage_rows = o.mailbox_step(pool, slots, w_gate_up, w_down, norm_weight=norm)
    assert_ffn_parity(o.gather(new_pool, slots), stage_rows, o.dense_fp32(normalized, w_gate_up, w_down))


@pytest.mark.parametrize("rows,gate_up", [(3, "split"), (12, "resident"), (33, "tile")])
def test_fp16_bad_slot_is_dropped(device, rows, gate_up):
    # A slot outside the mailbox: the row is staged as fp16 quiet NaNs by whichever gather
    # the step takes (fused into the split or resident kernel, or the separate gather
    # launch before the tiles), its output is dropped, the fault bit is raised, and the
    # other rows are their own FFN.
    hidden, intermediate, pool_rows = 1024, 3072, 64
    assert _native.dense_gate_up_variant(rows, hidden, intermediate).startswith(gate_up)
    print(f"fp16 bad slot rows={rows}", flush=True)
    pool = o.generate_hidden_states(pool_rows, hidden, 81).half()
    w_gate_up, w_down, norm_weight = _fp16_layer(hidden, intermediate, 82)
    good = o.generate_slots(pool_rows, rows, 83)
    bad = good.copy()
    bad[rows // 2] = pool_rows + 1
    with FfnAgent(device) as agent:
        agent.register_layer(
            instance_index=0, layer_ordinal=0, norm_weight=to_device(norm_weight, device),
            weights=DenseFfnWeights.from_tensors(to_device(w_gate_up, device), to_device(w_down, device)),
        )
        agent.materialize(maximum_row_capacity=64)
        pool_gpu = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(bad, device))
        with pytest.raises(FfnHealthError):
            agent.check_health()
    _check(pool_gpu, pool, np.delete(good, rows // 2), w_gate_up, w_down, norm_weight)


@pytest.mark.parametrize("mode", ("direct", "mailbox", "lane_stream"))
def test_fp16_ffn_shim(device, mode):
    # The shim takes the attached arena's payload dtype; a bf16 tensor is refused (the
    # reference's dtype check, instance.cpp:104-105).
    hidden, intermediate = 1024, 3072
    w_gate_up, w_down, _ = _fp16_layer(hidden, intermediate, 91)
    agent = FfnAgent(device)
    try:
        agent.register_layer(
            instance_index=0, layer_ordinal=0,
            weights=DenseFfnWeights.from_tensors(to_device(w_gate_up, device), to_device(w_down, device)),
        )
        agent.materialize(maximum_row_capacity=64)
        attach(agent, mailbox=mode != "direct", lane_stream=mode == "lane_stream")
        for rows in (1, 13, 64):
            x = o.generate_hidden_states(rows, hidden, 92 + rows).half()
            out = ffn_shim(to_device(x, device), None, DECODE)
            torch.cuda.synchronize()
            assert out.dtype is torch.float16
            assert_ffn_parity(out.cpu(), o.dense_partial_reference(x, w_gate_up, w_down),
                              o.dense_fp32(x, w_gate_up, w_down))
        with pytest.raises(RuntimeError, match="dtype"):
            ffn_shim(torch.zeros((4, hidden), dtype=torch.bfloat16, device=device), None, DECODE)
    finally:
        detach()
        agent.close()


@pytest.mark.parametrize("dtype,nan_bits", [(torch.float16, F16_NAN), (torch.bfloat16, 0x7FC0)])
def test_canonical_failure_fills_payload_nan(device, dtype, nan_bits):
    # A request after a published failure is answered with static_cast<Scalar>(NAN) in every
    # output element (instance.cu:28-31, instance_test.cu:97-115): the payload dtype's quiet
    # NaN, fp16 0x7e00 and bf16 0x7fc0.
    from crosspool_amd.ffn import ResultCode
    from crosspool_amd.transport import TransportResident

    with TransportResident(device, [(3, 1)]) as transport:
        transport.publish_failure(0, ResultCode.PROTOCOL_MISMATCH)
        output = torch.ones((3, 5), dtype=dtype, device=device)
        transport.submit(0, 3, DECODE)
        transport.complete(0, output)
        torch.cuda.synchronize()
        assert bool((output.cpu().view(torch.int16) == nan_bits).all())
