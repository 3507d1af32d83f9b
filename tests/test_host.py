"""Host logic and the C-ABI boundary without a GPU.

Covers the Python mirror of the reference interface (capacity buckets,
workspace geometry, signatures, request metadata, enums) and that the HIP
library loads and exports every symbol ``include/xpool_amd.h`` declares.  The
only native calls made are argument-validation paths that return before any
HIP call, plus pure queries.
"""

from __future__ import annotations

import ctypes
import re

import pytest
import torch

from crosspool_amd import _native
from crosspool_amd.execution import (
    DenseFfnExecutionSignature,
    WorkspaceLayout,
    dense_signatures,
    derive_payload_row_capacities,
    select_capacity,
)
from crosspool_amd.ffn import (
    DpRowLayout,
    ForwardMode,
    GateTransform,
    GateUpOrder,
    LayerKind,
    OutputRequirement,
    ResultCode,
    SiluActivation,
    activation_arguments,
)
from crosspool_amd.transport import FfnRequestMetadata


def _declared_functions() -> list[str]:
    text = _native.HEADER_PATH.read_text()
    return sorted(set(re.findall(r"^(?:int|size_t)\s+(xp_\w+)\s*\(", text, flags=re.MULTILINE)))


def test_library_exports_every_declared_symbol():
    lib = _native.library()
    declared = _declared_functions()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), f"{name} missing from {_native.LIBRARY_PATH}"
    assert set(declared) == set(_native.SIGNATURES), "ctypes signatures and header disagree"
    assert lib.xp_abi_version() == 2  # the MoE calls take payload dtypes, biases and activations


def test_header_enums_match_the_reference_values():
    # src/cext-include/xpool/ffn.hpp:15-54
    text = _native.HEADER_PATH.read_text()
    expected = {
        "XP_FORWARD_PREFILL": ForwardMode.PREFILL, "XP_FORWARD_DECODE": ForwardMode.DECODE,
        "XP_FORWARD_IDLE": ForwardMode.IDLE, "XP_OUTPUT_PER_RANK_COMPLETE": OutputRequirement.PER_RANK_COMPLETE,
        "XP_OUTPUT_GROUP_SUM_COMPLETE": OutputRequirement.GROUP_SUM_COMPLETE, "XP_DP_ROWS_NONE": DpRowLayout.NONE,
        "XP_DP_ROWS_UNIFORM_BY_RANK": DpRowLayout.UNIFORM_BY_RANK,
        "XP_DP_ROWS_PACKED_BY_RANK": DpRowLayout.PACKED_BY_RANK, "XP_RESULT_TIMEOUT": ResultCode.TIMEOUT,
        "XP_LAYER_DENSE": LayerKind.DENSE, "XP_LAYER_MOE": LayerKind.MOE,
    }
    for name, value in expected.items():
        match = re.search(rf"{name}\s*=\s*(\d+)", text)
        assert match and int(match.group(1)) == int(value), name
    assert (ForwardMode.PREFILL, ForwardMode.DECODE, ForwardMode.IDLE) == (1, 2, 4)


def test_capacity_buckets_match_reference():
    # tests/suites/unit/runtime/ffnagent/test_execution.py:18-24
    assert derive_payload_row_capacities(1) == (1,)
    assert derive_payload_row_capacities(5) == (1, 2, 4, 5)
    assert derive_payload_row_capacities(8) == (1, 2, 4, 8)
    assert derive_payload_row_capacities(4096)[-3:] == (1024, 2048, 4096)
    with pytest.raises(ValueError, match="positive"):
        derive_payload_row_capacities(0)
    with pytest.raises(TypeError):
        derive_payload_row_capacities(True)
    assert select_capacity((1, 2, 4, 5), 3) == 4
    with pytest.raises(ValueError):
        select_capacity((1, 2, 4, 5), 6)


def test_workspace_layout_matches_reference_known_answers():
    # test_execution.py:26-60: the gated CONCATENATED 4x16x8 plan needs 192 bytes, the
    # activated view starts 128 bytes in, a short or misaligned backing is refused.
    layout = WorkspaceLayout.from_regions(((torch.bfloat16, (4, 16)), (torch.bfloat16, (4, 8)), (torch.uint8, (0,))))
    assert layout.nbytes == 192
    backing = torch.empty(layout.nbytes, dtype=torch.uint8)
    projected, activated, _ = layout.views(backing)
    assert projected.data_ptr() == backing.data_ptr()
    assert activated.data_ptr() == backing.data_ptr() + 128
    assert projected.shape == (4, 16) and activated.shape == (4, 8)
    with pytest.raises(ValueError, match="layout needs 192"):
        layout.views(backing[:-1])
    misaligned = torch.empty(layout.nbytes + 1, dtype=torch.uint8)[1:]
    with pytest.raises(ValueError, match="16-byte boundary"):
        layout.views(misaligned)


@pytest.mark.parametrize("capacity,hidden,intermediate", [(1, 1024, 3072), (4096, 4096, 12288), (8, 5120, 3200), (3, 8, 8)])
def test_native_workspace_covers_signature_layout(capacity, hidden, intermediate):
    signature = DenseFfnExecutionSignature(torch.bfloat16, capacity, hidden, intermediate)
    native = _native.dense_workspace_bytes(capacity, hidden, intermediate)
    layout = signature.workspace_layout().nbytes
    down = _native.gemm_workspace_bytes(capacity, hidden, intermediate, False)
    # The partial sums of K-split projections follow the two regions, 256-byte aligned.  The
    # step's gate_up may differ from the kernel-level choice (at decode sizes it fuses the
    # gather into the stream kernel), so only the down partials are known here.
    assert native >= layout + down
    assert native == layout or native >= (layout + 255) // 256 * 256


def test_signature_validation():
    # bf16 and fp16 payloads (is_supported_payload_dtype, ffn.hpp:83-85); fp32 is refused
    DenseFfnExecutionSignature(torch.float16, 4, 16, 8)
    with pytest.raises(ValueError, match="bf16 or fp16"):
        DenseFfnExecutionSignature(torch.float32, 4, 16, 8)
    with pytest.raises(ValueError, match="multiples of 8"):
        DenseFfnExecutionSignature(torch.bfloat16, 4, 12, 8)
    with pytest.raises(ValueError, match="positive"):
        DenseFfnExecutionSignature(torch.bfloat16, 0, 16, 8)
    with pytest.raises(ValueError, match="default SiLU"):
        DenseFfnExecutionSignature(torch.bfloat16, 4, 16, 8, activation=SiluActivation(alpha=1.3))
    signatures = dense_signatures(hidden_size=1024, local_intermediate_size=3072, maximum_row_capacity=5)
    assert [s.payload_row_capacity for s in signatures] == [1, 2, 4, 5]
    assert len(set(signatures)) == 4  # hashable GraphTemplate keys


def test_request_metadata_validation():
    # src/xpool/transport.py:32-42
    FfnRequestMetadata(0, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE, DpRowLayout.NONE)
    with pytest.raises(ValueError):
        FfnRequestMetadata(-1, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE, DpRowLayout.NONE)
    with pytest.raises(ValueError):
        FfnRequestMetadata(True, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE, DpRowLayout.NONE)
    with pytest.raises(TypeError):
        FfnRequestMetadata(0, 2, OutputRequirement.PER_RANK_COMPLETE, DpRowLayout.NONE)
    with pytest.raises(TypeError):
        FfnRequestMetadata(0, ForwardMode.DECODE, 1, DpRowLayout.NONE)
    with pytest.raises(TypeError):
        FfnRequestMetadata(0, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE, 0)


def test_gate_up_order_and_activation_arguments():
    gate, up = GateUpOrder.INTERLEAVED.row_indices(width=8, start=2, length=3)
    assert list(range(16))[gate] == [4, 6, 8] and list(range(16))[up] == [5, 7, 9]
    gate, up = GateUpOrder.CONCATENATED.row_indices(width=8, start=2, length=3)
    assert list(range(16))[gate] == [2, 3, 4] and list(range(16))[up] == [10, 11, 12]
    assert activation_arguments(SiluActivation(), GateTransform()) == (1.0, 0.0, 0.0)
    assert activation_arguments(SiluActivation(1.3), GateTransform(4.0, -0.5)) == (1.3, 4.0, -0.5)
    with pytest.raises(ValueError):
        SiluActivation(alpha=0.0)
    with pytest.raises(ValueError):
        GateTransform(limit=-1.0)


def test_moe_experts_rejects_buffer_ranges_past_2_gib():
    lib = _native.library()
    f = ctypes.c_float
    # 2^21 rows of 1024 bf16 = 4 GiB of token rows: refused before any pointer is used.
    status = lib.xp_moe_experts(None, 1 << 21, 1024, 256, 8, 2, None, None, None, None, None, None, f(1.0),
                                _native.XP_ACTIVATION_SILU, 0, f(1.0), f(0.0), f(0.0), _native.XP_DTYPE_BF16, None,
                                None, 0, None)
    assert status == _native.XP_ERROR_INVALID_ARGUMENT
    assert "2 GiB" in _native.last_error()
    # An expert of 2 x 32768 x 16384 bf16 gate_up rows is past one range as well.
    status = lib.xp_moe_experts(None, 4, 16384, 32768, 8, 2, None, None, None, None, None, None, f(1.0),
                                _native.XP_ACTIVATION_SILU, 0, f(1.0), f(0.0), f(0.0), _native.XP_DTYPE_BF16, None,
                                None, 0, None)
    assert status == _native.XP_ERROR_INVALID_ARGUMENT
    # An activation outside SiLU / ReLU / GELU, and the tanh form on anything but GELU.
    status = lib.xp_moe_experts(None, 4, 1024, 256, 8, 2, None, None, None, None, None, None, f(1.0), 0, 0,
                                f(1.0), f(0.0), f(0.0), _native.XP_DTYPE_BF16, None, None, 0, None)
    assert status == _native.XP_ERROR_INVALID_ARGUMENT and "activation" in _native.last_error()
    status = lib.xp_moe_experts(None, 4, 1024, 256, 8, 2, None, None, None, None, None, None, f(1.0),
                                _native.XP_ACTIVATION_RELU, 1, f(1.0), f(0.0), f(0.0), _native.XP_DTYPE_BF16, None,
                                None, 0, None)
    assert status == _native.XP_ERROR_INVALID_ARGUMENT


def test_dense_step_rejects_mailbox_pools_past_2_gib():
    # The fused gathers address the whole mailbox pool through one 32-bit buffer resource:
    # 262144 slots of 4096 bf16 are 2 GiB and must be refused before any pointer is used.
    lib = _native.library()
    status = lib.xp_dense_step(None, None, 1 << 18, None, 1, 4096, 12288, None, None, None, ctypes.c_float(1e-6),
                               None, 0, None, None)
    assert status == _native.XP_ERROR_INVALID_ARGUMENT
    assert "2 GiB" in _native.last_error()
    status = lib.xp_dense_step_static(None, None, 1 << 18, None, 1, 4096, 12288, None, None, None,
                                      ctypes.c_float(1e-6), None, None)
    assert status == _native.XP_ERROR_INVALID_ARGUMENT
    assert "2 GiB" in _native.last_error()


def test_dense_projections_past_one_buffer_range_take_the_tile_kernel():
    # The split and stream kernels address the whole weight matrix through one 32-bit buffer
    # resource; a gate_up of 2 x 53248 x 16384 bf16 (3.5 GB, a TP-1 shard of a very wide model)
    # or a 4 GiB down must go to the tile kernel, whose resources span one tile, at every
    # decode size, and the Dense step's gate_up must not fuse the gather into a stream kernel.
    for rows in (1, 4, 8, 16):
        assert _native.gemm_variant(rows, 2 * 53248, 16384, True).startswith("tile_gated")
        assert _native.gemm_variant(rows, 16384, 131072, False).startswith("tile")
    # Just below one range the decode kernels stay eligible.
    assert _native.gemm_variant(1, 2 * 8192, 65528, True).startswith(("split", "stream"))
    # The tile kernel's per-tile ranges are bounded through the intermediate size.
    assert _native.dense_workspace_bytes(16, 16384, 53248) > 0
    offsets = (ctypes.c_size_t * 5)()
    assert _native.library().xp_dense_workspace_layout(16, 1024, (1 << 21) + 8, offsets) == (
        _native.XP_ERROR_INVALID_ARGUMENT
    )
    assert "2^21" in _native.last_error()


def test_dense_workspace_layout_matches_the_region_rules():
    # Batch at 0, activated after it (16-byte aligned), fp32 partials 256-byte aligned after
    # that when a projection at this capacity splits K, total = xp_dense_workspace_bytes.
    for capacity, hidden, intermediate in ((1, 1024, 3072), (32, 4096, 12288), (2048, 4096, 12288), (3, 1032, 1000)):
        batch, activated, gate_up, down, total = _native.dense_workspace_layout(capacity, hidden, intermediate)
        assert batch == 0
        assert activated == (capacity * hidden * 2 + 15) // 16 * 16
        assert total == _native.dense_workspace_bytes(capacity, hidden, intermediate)
        if gate_up == total:
            assert down == total and total == activated + capacity * intermediate * 2
        else:
            assert gate_up % 256 == 0 and gate_up >= activated + capacity * intermediate * 2
            assert gate_up <= down <= total
    # Qwen3-8B at 32 rows splits down over 8 K ranges: 8 x 32 x 4096 fp32 partials.
    _, _, gate_up, down, total = _native.dense_workspace_layout(32, 4096, 12288)
    assert total - down == 8 * 32 * 4096 * 4 and gate_up == down


def test_moe_step_workspace_layout_and_descriptor_checks():
    # Regions in order, each 256-byte aligned: batch [C, H] bf16, Router workspace (logits
    # first), routed ids / weights [C, routed_topk], final ids / weights [C, effective] only
    # with shared experts, then the Experts workspace at C rows; total = the bytes query.
    from crosspool_amd.moe import MoeLayerSpec

    def align(value):
        return (value + 255) // 256 * 256

    for capacity, hidden, intermediate, routed, shared, topk in ((1, 2048, 768, 128, 0, 8), (37, 512, 256, 16, 2, 3)):
        spec = MoeLayerSpec(routed_expert_count=routed, routed_topk=topk, shared_expert_count=shared)
        signature = spec.signature(hidden_size=hidden, local_intermediate_size=intermediate,
                                   payload_row_capacity=capacity)
        assert signature.effective_topk == topk + shared and signature.expert_count == routed + shared
        assert signature.routing_storage_bytes == capacity * (topk + shared) * 8
        desc = signature.native_descriptor()
        batch, logits, rid, rw, fid, fw, experts, total = _native.moe_step_workspace_layout(desc, capacity)
        assert batch == 0 and logits == align(capacity * hidden * 2)
        router_bytes = _native.library().xp_moe_router_workspace_bytes(capacity, hidden, routed, 1)
        assert rid == align(logits + router_bytes) and rw == align(rid + capacity * topk * 4)
        if shared:
            assert fid == align(rw + capacity * topk * 4) and fw == align(fid + capacity * (topk + shared) * 4)
            assert experts == align(fw + capacity * (topk + shared) * 4)
        else:
            assert (fid, fw) == (rid, rw) and experts == align(rw + capacity * topk * 4)
        moe_bytes = _native.library().xp_moe_workspace_bytes(capacity, hidden, intermediate, routed + shared,
                                                             topk + shared)
        assert total == align(experts + moe_bytes) == _native.moe_step_workspace_bytes(desc, capacity)

    spec = MoeLayerSpec(routed_expert_count=8, routed_topk=2)
    good = spec.signature(hidden_size=256, local_intermediate_size=128, payload_row_capacity=4).native_descriptor()
    for field, value, message in (
        ("hidden", 260, "multiples of 8"),
        ("routed_experts", 9, "routed experts"),
        ("routed_topk", 9, "topk"),
        ("algorithm", 3, "algorithm"),
        ("precision", 0, "precision"),
        ("routed_scaling_factor", 0.0, "scaling"),
        ("alpha", -1.0, "alpha"),
        ("limit", -1.0, "limit"),
        ("activation", 0, "activation"),
        ("approximate_tanh", 1, "tanh"),
        ("biases", 4, "biases"),
    ):
        bad = _native.MoeLayerDesc.from_buffer_copy(good)
        setattr(bad, field, value)
        assert _native.moe_step_workspace_bytes(bad, 4) == 0
        with pytest.raises(_native.NativeError, match=message):
            _native.moe_step_workspace_layout(bad, 4)
    with pytest.raises(_native.NativeError, match="capacity must be positive"):
        _native.moe_step_workspace_layout(good, 0)
    with pytest.raises(ValueError, match="TopK"):
        MoeLayerSpec(routed_expert_count=4, routed_topk=5)
    with pytest.raises(ValueError, match="1024"):
        MoeLayerSpec(routed_expert_count=1024, routed_topk=8, shared_expert_count=1)
    lib = _native.library()
    assert lib.xp_moe_layer_register(None, 0, 0, ctypes.byref(good), None, None, None, None, None, None, None,
                                     1e-6) != 0
    assert lib.xp_moe_template_capture(None, ctypes.byref(good), 4) != 0


def test_abi_rejects_invalid_arguments_before_touching_the_device():
    lib = _native.library()
    p = ctypes.c_void_p
    # hidden not a multiple of 8
    assert lib.xp_gather_rmsnorm(p(16), 4, 12, p(16), 2, None, 1e-6, p(16), None, None) == _native.XP_ERROR_INVALID_ARGUMENT
    assert "multiple of 8" in _native.last_error()
    # misaligned rows
    assert lib.xp_scatter(p(8), 1, 8, p(16), p(16), 4, None, None) == _native.XP_ERROR_INVALID_ARGUMENT
    # overlapping copy ranges
    assert lib.xp_copy_bytes(p(4096), p(4100), 64, None) == _native.XP_ERROR_INVALID_ARGUMENT
    assert "overlap" in _native.last_error()
    # zero rows are no-ops; zero-length copies accept null pointers
    assert lib.xp_gather_rmsnorm(None, 0, 8, None, 0, None, 1e-6, None, None, None) == _native.XP_OK
    assert lib.xp_copy_bytes(None, None, 0, None) == _native.XP_OK
    # SiLU alpha must be positive
    assert lib.xp_gemm_gate_up_silu(p(16), 1, 16, p(16), 8, p(16), 0.0, 0.0, 0.0, None, 0, None) == _native.XP_ERROR_INVALID_ARGUMENT
    # a sliced projection without its scratch
    assert lib.xp_gemm_down(p(16), 32, 12288, p(16), 4096, p(16), None, 32, None, 0, None) == _native.XP_ERROR_CAPACITY
    assert "xp_gemm_workspace_bytes" in _native.last_error()
    # null handles
    assert lib.xp_layer_register(None, 0, 0, 16, 8, _native.XP_DTYPE_BF16, p(16), p(16), None, 1e-6) == (
        _native.XP_ERROR_INVALID_ARGUMENT
    )
    assert lib.xp_replay(None, 0, 0, 1, p(16), p(16), 1, p(16), None) == _native.XP_ERROR_INVALID_ARGUMENT
    assert lib.xp_dense_workspace_bytes(0, 16, 8) == 0
    with pytest.raises(_native.NativeError) as error:
        _native.check(_native.XP_ERROR_CAPACITY, "probe")
    assert error.value.status == _native.XP_ERROR_CAPACITY


def test_gemm_variant_selection():
    # decode sizes: the split, stream or resident kernel, never a tile
    for rows in (1, 2, 4, 8, 9, 16):
        for n, k, gated in ((24576, 4096, True), (4096, 12288, False), (19456, 2560, True), (2560, 9728, False)):
            assert _native.gemm_variant(rows, n, k, gated).startswith(("split", "stream", "resident"))
    assert _native.gemm_variant(1, 4096, 12288, False) == "split_t8_k8"
    # 9 to 16 rows: the resident kernel where its weight rows fill the grid (N >= 2048),
    # K split over the grid when one part of 8 waves x 4 chunks does not cover it
    assert _native.gemm_variant(16, 24576, 4096, True) == "resident_gated_t16_c4"
    assert _native.gemm_variant(9, 12288, 6000, True) == "resident_gated_t16_c3_p2"
    assert _native.gemm_workspace_bytes(9, 12288, 6000, True) == 2 * 9 * 12288 * 4
    assert _native.gemm_variant(16, 5120, 3200, False) == "resident_t16_c4"
    assert _native.gemm_workspace_bytes(16, 5120, 3200, False) == 0
    assert _native.gemm_variant(16, 6400, 5120, True) == "stream_gated_t16"
    # Qwen3-4B and Qwen3-0.6B down: K ranges of whole 128-wide chunks let the split kernel
    # take 8 ranges (160 and 64 workgroups), with no scratch
    assert _native.gemm_variant(1, 2560, 9728, False) == "split_t8_k8"
    assert _native.gemm_variant(1, 1024, 3072, False) == "split_t8_k8"
    assert _native.gemm_workspace_bytes(1, 2560, 9728, False) == 0
    assert _native.gemm_variant(17, 24576, 4096, True) == "tile_gated_64x64"
    assert _native.gemm_variant(128, 6144, 1024, True) == "tile_gated_64x64"  # 96 tiles of 64 x 128
    assert _native.gemm_variant(128, 24576, 4096, True) == "tile_gated_128x128"
    assert _native.gemm_variant(64, 4096, 12288, False).startswith("tile_64x128_k")
    assert _native.gemm_workspace_bytes(1, 24576, 4096, True) == 0
    # 9 to 16 rows: the split kernel with two token groups where its modelled cost is lower
    # (Qwen3-0.6B down; its K ranges are summed in LDS, no scratch), else the stream kernel
    # (Qwen3-8B down: 8 K slices of 1536, whose fp32 partials the reduction launch sums)
    assert _native.gemm_variant(16, 1024, 3072, False) == "split_t16_k8"
    assert _native.gemm_workspace_bytes(16, 1024, 3072, False) == 0
    assert _native.gemm_variant(16, 1536, 8960, False) == "stream_t16"
    assert _native.gemm_variant(16, 4096, 12288, False) == "stream_t16"
    assert _native.gemm_workspace_bytes(16, 4096, 12288, False) == 8 * 16 * 4096 * 4
    assert _native.gemm_variant(2048, 24576, 4096, True) == "tile_gated_256x256"
    assert _native.gemm_variant(4096, 4096, 12288, False).startswith("tile")
    assert _native.gemm_workspace_bytes(2048, 24576, 4096, True) == 0


def test_dense_step_fuses_the_gather_at_decode_sizes():
    # Qwen3-0.6B gate_up up to 8 rows: the split kernel stages the gathered, normalised rows
    # itself (one round of workgroups).  Qwen3-1.7B / 4B / 8B up to 8 rows (768 / 608 / 1536
    # units): the persistent split kernel, two workgroups per CU, each gathering once.  K past
    # 4096 (the 32B TP shard's 5120) does not fit the split kernel's staging, and past 16 rows
    # the gather is a launch of its own.
    for rows in (1, 4, 8):
        assert _native.dense_gate_up_variant(rows, 1024, 3072) == "split_gated_t8_k4+gather"
        assert _native.dense_gate_up_variant(rows, 2048, 6144) == "split_gated_t8_k8_persistent+gather"
        assert _native.dense_gate_up_variant(rows, 2560, 9728) == "split_gated_t8_k4_persistent+gather"
        assert _native.dense_gate_up_variant(rows, 4096, 12288) == "split_gated_t8_k8_persistent+gather"
        assert "+gather" not in _native.dense_gate_up_variant(rows, 5120, 3200)
    # 9 to 16 rows: the resident kernel gathers and normalises the rows itself when one part
    # covers K (not the 32B TP shard's 5120, which keeps a separate gather)
    for rows in (9, 16):
        assert _native.dense_gate_up_variant(rows, 4096, 12288) == "resident_gated_t16_c4+gather"
        assert _native.dense_gate_up_variant(rows, 1024, 3072) == "resident_gated_t16_c1+gather"
        assert "+gather" not in _native.dense_gate_up_variant(rows, 5120, 3200)
    # 17 to 32 rows: four token groups where gate_up has at least 16384 weight rows (Qwen3-4B
    # and 8B), the tile kernels on a separate gather below that (Qwen3-1.7B)
    for rows in (17, 32):
        assert _native.dense_gate_up_variant(rows, 4096, 12288) == "resident_gated_t32_c4+gather"
        assert _native.dense_gate_up_variant(rows, 2560, 9728) == "resident_gated_t32_c3+gather"
        assert "+gather" not in _native.dense_gate_up_variant(rows, 2048, 6144)
    assert _native.dense_gate_up_variant(33, 4096, 12288) == "tile_gated_64x128"
    # kernel-level projections (no gather) keep the 16-row ceiling
    assert _native.gemm_variant(32, 24576, 4096, True) == "tile_gated_64x64"
    assert _native.dense_gate_up_variant(2048, 4096, 12288) == "tile_gated_256x256"


def test_short_reductions_never_take_the_persistent_split():
    # With K <= 128 no K range reaches two 128-wide chunks: the persistent split kernel has no
    # split to walk and must not be chosen (it would read nothing and store zeros), however
    # many units the intermediate gives it.
    for rows in range(1, 9):
        for hidden in (64, 128):
            variant = _native.dense_gate_up_variant(rows, hidden, 32768)
            assert "persistent" not in variant, (rows, hidden, variant)
    # one K range of two chunks is enough again
    assert "persistent" in _native.dense_gate_up_variant(1, 256, 32768)


def test_operator_scratch_serves_every_live_row_count_up_to_the_plan():
    # A kernel-level projection chooses its kernel at the live row count, and a smaller count
    # can take more K ranges than the plan's capacity: the plan's scratch is the largest need.
    planned = _native.gemm_workspace_bytes_upto(117, 1024, 3072, False)
    assert planned >= _native.gemm_workspace_bytes(59, 1024, 3072, False) > _native.gemm_workspace_bytes(
        117, 1024, 3072, False
    )
    assert planned == max(_native.gemm_workspace_bytes(r, 1024, 3072, False) for r in range(1, 118))


def test_k_split_tiles_fill_the_chip_and_size_their_partials():
    # Qwen3-8B down at 256 rows has only 16 to 64 weight x token tiles: K is split so that
    # the grid covers the 256 CUs, and each range leaves an fp32 partial tile in scratch.
    name = _native.gemm_variant(256, 4096, 12288, False)
    shape, split = name.split("_")[1], int(name.rsplit("_k", 1)[1])
    bm, bn = (int(v) for v in shape.split("x"))
    tiles = -(-256 // bm) * (4096 // bn)
    assert tiles < 256 <= tiles * split
    assert _native.gemm_workspace_bytes(256, 4096, 12288, False) == split * 256 * 4096 * 4
    # with a K of one slab there is nothing to split
    assert "_k" not in _native.gemm_variant(300, 128, 64, False)


def test_column_split_fills_the_last_round():
    # Qwen3-32B TP shard at 8192 rows: 32 token tiles x 25 weight tiles of 256 x 256 would be
    # 3.125 rounds of one tile per CU.  The first 24 weight tiles (768 tiles, 3 whole rounds)
    # stay on 256 x 256 and the last 256 weight rows go to a second launch of 64 x 128 tiles
    # (256 tiles: one more round of small tiles instead of a round one eighth full).
    name = _native.gemm_variant(8192, 6400, 5120, True)
    assert name == "tile_gated_256x256+64x128_n256"
    main_weight_tiles = (6400 - 256) // 256
    assert (8192 // 256) * main_weight_tiles % 256 == 0
    assert (8192 // 64) * (256 // 128) == 256
    # no K split in either launch: no scratch
    assert _native.gemm_workspace_bytes(8192, 6400, 5120, True) == 0
    # Whole rounds already: one shape.
    assert "+" not in _native.gemm_variant(2048, 24576, 4096, True)
    assert "+" not in _native.gemm_variant(4096, 4096, 12288, False)
    # The first launch is always the 256 x 256 tile (a 256 x 128 first launch measured slower).
    for rows, n, k in ((512, 24576, 4096), (2048, 5120, 3200), (512, 19456, 2560)):
        for gated in (True, False):
            name = _native.gemm_variant(rows, n, k, gated)
            assert "+" not in name or "_256x256+" in name


def test_ffn_shim_requires_an_attachment():
    from crosspool_amd.ops import ffn_shim

    metadata = FfnRequestMetadata(0, ForwardMode.PREFILL, OutputRequirement.PER_RANK_COMPLETE, DpRowLayout.NONE)
    with pytest.raises(RuntimeError, match="no attached"):
        ffn_shim(torch.zeros((2, 16), dtype=torch.bfloat16), None, metadata)


def test_transport_entry_points_validate_before_any_device_call():
    lib = _native.library()
    handle = ctypes.c_void_p()
    capacities = (ctypes.c_int64 * 1)(4)
    dp_sizes = (ctypes.c_int32 * 1)(1)
    assert lib.xp_transport_create(0, 0, capacities, dp_sizes, ctypes.byref(handle)) == _native.XP_ERROR_INVALID_ARGUMENT
    assert "1 to 1024 arenas" in _native.last_error()
    bad_dp = (ctypes.c_int32 * 1)(65)
    assert lib.xp_transport_create(0, 1, capacities, bad_dp, ctypes.byref(handle)) == _native.XP_ERROR_INVALID_ARGUMENT
    assert lib.xp_transport_submit(None, 0, 1, 0, 2, 1, 0, None, 0, 0, None) == _native.XP_ERROR_INVALID_ARGUMENT
    assert lib.xp_transport_evaluate(None, 0, None, None) == _native.XP_ERROR_INVALID_ARGUMENT
    assert lib.xp_transport_complete(None, 0, None, 0, _native.XP_DTYPE_BF16, 0, None) == _native.XP_ERROR_INVALID_ARGUMENT
    assert lib.xp_transport_probe(None, 0, 0, None, 0) == _native.XP_ERROR_INVALID_ARGUMENT
    assert lib.xp_transport_destroy(None) == _native.XP_OK


def test_integration_argtypes_match_the_library():
    # Every ctypes binding INTEGRATION.md shows a maintainer must match the signature table
    # the package binds the library with (names and argument types, in order).
    import re
    from pathlib import Path

    doc = (Path(__file__).resolve().parents[1] / "INTEGRATION.md").read_text()
    kinds = {"P": ctypes.c_void_p, "INT": ctypes.c_int, "I64": ctypes.c_int64, "F32": ctypes.c_float,
             "SIZE": ctypes.c_size_t}
    checked = 0
    for match in re.finditer(r"lib\.(xp_\w+)\.argtypes = \[", doc):
        name = match.group(1)
        depth, body = 0, ""
        for ch in doc[match.end() - 1:]:
            body += ch
            depth += ch == "["
            depth -= ch == "]"
            if depth == 0:
                break
        body = re.sub(r"#[^\n]*", "", body)[1:-1]
        tokens = [t.strip() for t in re.split(r",(?![^()]*\))", body.replace("\n", " ")) if t.strip()]
        expected = _native.SIGNATURES[name][1]
        assert len(tokens) == len(expected), name
        for token, want in zip(tokens, expected):
            if token in kinds:
                assert kinds[token] is want, (name, token, want)
            else:
                assert token.startswith("ctypes.POINTER("), (name, token)
        checked += 1
    assert checked >= 20
