"""Pin the CPU oracle (no GPU).

Each oracle function is checked against something that does not restate its
own formula: the reference's known answers, the independent C restatement,
exact rational brute force, closed forms and invariants -- chosen so a
dropped term, a swapped Gate/Up, a missing rounding stage or a transposed
operand fails at least one check.
"""

from __future__ import annotations

import math
import struct
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import ffn_oracle as o

from conftest import GOLDEN_DIR


# --------------------------------------------------------------- bf16 rounding
def _bf16_round_fraction(value: Fraction) -> float:
    """Exact round-to-nearest-even of a rational to bf16 (8 significant bits), via fp32 first.

    torch converts fp64 -> bf16 through fp32; a Fraction is first rounded to the
    nearest double (exact for the test magnitudes), then to fp32, then to bf16.
    """

    as_float32 = struct.unpack("f", struct.pack("f", float(value)))[0]
    return _bf16_round_float(as_float32)


def _round_half_even(value: Fraction) -> int:
    floor = math.floor(value)
    remainder = value - floor
    if remainder > Fraction(1, 2) or (remainder == Fraction(1, 2) and floor % 2 == 1):
        floor += 1
    return floor


def _bf16_round_float(value: float) -> float:
    if value == 0 or not math.isfinite(value):
        return value
    _, exponent = math.frexp(value)  # value = m * 2**exponent, 0.5 <= |m| < 1
    # 8 significant bits for normals; below 2^-126 the spacing is fixed at 2^-133.
    quantum = Fraction(2) ** max(exponent - 8, -133)
    return float(_round_half_even(Fraction(value) / quantum) * quantum)


def test_bf16_rounding_matches_c_restatement_on_edge_patterns():
    values = np.array(
        [1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, -1.0 - 2**-8, 3.999, 1e-30, -2.5e-39, 65504.0, 0.0, -0.0], dtype=np.float32
    )
    c_bits = c_oracle.bf16_from_float(values)
    torch_bits = o.bf16_bits(torch.from_numpy(values).to(torch.bfloat16))
    assert np.array_equal(c_bits, torch_bits)
    for value, bits in zip(values, torch_bits):
        assert _bf16_round_float(float(value)) == struct.unpack("f", struct.pack("I", int(bits) << 16))[0]


def test_fp64_to_bf16_rounds_through_fp32_like_the_reference():
    # qualification.py:309-314 converts fp64 sums with torch's .to(bf16), which rounds through
    # fp32: 1 + 2^-8 + 2^-40 ties to 1.0 instead of rounding up.
    value = torch.tensor([1 + 2**-8 + 2**-40], dtype=torch.float64)
    assert float(value.to(torch.bfloat16)) == 1.0
    assert _bf16_round_fraction(Fraction(1) + Fraction(1, 256) + Fraction(1, 2**40)) == 1.0


# --------------------------------------------------------------- transport
COPY_CASES = [(32, 16, 128), (7, 3, 128), (32, 16, 127), (0, 0, 0)]


@pytest.mark.parametrize("dst_offset,src_offset,count", COPY_CASES)
def test_copy_bytes_reference_cases(dst_offset, src_offset, count):
    # tests/suites/cext/utils/cooperative_test.cu:40-111: pattern (i*17+3) % 251, sentinel 0xa5.
    source = np.array([(i * 17 + 3) % 251 for i in range(256)], dtype=np.uint8)
    destination = np.full(256, 0xA5, dtype=np.uint8)
    o.copy_bytes(destination[dst_offset : dst_offset + count], source[src_offset : src_offset + count])
    c_destination = np.full(256, 0xA5, dtype=np.uint8)
    lib = c_oracle.library()
    assert lib.xpo_copy_bytes(
        c_destination.ctypes.data + dst_offset, count, source.ctypes.data + src_offset, count
    ) == 0
    for index in range(256):
        copied = dst_offset <= index < dst_offset + count
        expected = source[src_offset + index - dst_offset] if copied else 0xA5
        assert destination[index] == expected
        assert c_destination[index] == expected


def test_copy_bytes_rejects_size_mismatch():
    with pytest.raises(ValueError):
        o.copy_bytes(np.zeros(4, np.uint8), np.zeros(5, np.uint8))
    assert c_oracle.library().xpo_copy_bytes(np.zeros(4, np.uint8).ctypes.data, 4, np.zeros(5, np.uint8).ctypes.data, 5) == -1


def test_gather_scatter_closed_forms_and_c_restatement():
    pool = o.generate_hidden_states(40, 24, 17)
    slots = np.array([39, 0, 7, 12, 33], dtype=np.int32)
    gathered = o.gather(pool, slots)
    for row, slot in enumerate(slots):
        assert torch.equal(gathered[row].view(torch.int16), pool[slot].view(torch.int16))
    assert torch.equal(c_oracle.gather(pool, slots).view(torch.int16), gathered.view(torch.int16))
    values = o.generate_hidden_states(5, 24, 23)
    scattered = o.scatter(pool, slots, values)
    assert torch.equal(c_oracle.scatter(pool, slots, values).view(torch.int16), scattered.view(torch.int16))
    untouched = np.setdiff1d(np.arange(40), slots)
    assert torch.equal(scattered[untouched].view(torch.int16), pool[untouched].view(torch.int16))
    # identity slots: the reference's prefix copy (instance.cu:83-84)
    assert torch.equal(o.gather(pool, np.arange(9)).view(torch.int16), pool[:9].view(torch.int16))
    # round trip: scatter(gather(slots)) restores the pool bit-for-bit
    assert torch.equal(o.scatter(pool, slots, gathered).view(torch.int16), pool.view(torch.int16))
    with pytest.raises(IndexError):
        o.gather(pool, np.array([40]))
    with pytest.raises(ValueError):
        o.scatter(pool, np.array([1, 1]), values[:2])


# --------------------------------------------------------------- RMSNorm
def test_rmsnorm_matches_c_restatement_and_fp64_brute_force():
    x = o.generate_hidden_states(64, 1024, 17)
    _, _, weight = o.generate_layer(1024, 8, 18)
    result = o.rmsnorm(x, weight, 1e-6)
    assert torch.equal(result.view(torch.int16), c_oracle.rmsnorm(x, weight, 1e-6).view(torch.int16))
    x64 = x.double()
    brute = (x64 / torch.sqrt((x64 * x64).mean(-1, keepdim=True) + 1e-6) * weight.double()).to(torch.bfloat16)
    differ = (result.float() - brute.float()).abs()
    assert bool((differ <= o.bf16_ulp(brute)).all())
    assert float((result.view(torch.int16) == brute.view(torch.int16)).float().mean()) > 0.99


def test_rmsnorm_closed_forms():
    hidden = 256
    weight = torch.ones(hidden, dtype=torch.bfloat16)
    x = torch.zeros((3, hidden), dtype=torch.bfloat16)
    x[0] = -3.0  # constant row -> -1 after normalisation
    x[1] = 1e-3  # eps not negligible: x / sqrt(x^2 + eps)
    out = o.rmsnorm(x, weight, 1e-6)
    assert torch.equal(out[0].float(), torch.full((hidden,), -1.0))
    v = float(x[1, 0])
    assert float(out[1, 0]) == pytest.approx(v / math.sqrt(v * v + 1e-6), rel=2**-8)
    assert torch.equal(out[2].float(), torch.zeros(hidden))
    # eps dropped would give exactly 1.0 for the small constant row:
    assert float(out[1, 0]) < 0.8
    # weight scales each column
    w = torch.arange(1, hidden + 1, dtype=torch.float32).to(torch.bfloat16)
    scaled = o.rmsnorm(x[:1], w, 1e-6)
    assert torch.equal(scaled[0].float(), (-w.float()).to(torch.bfloat16).float())


# --------------------------------------------------------------- Dense / SiLU
def _fraction_dense(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor) -> tuple[list, list]:
    """Pure-Python exact brute force of qualification.py:290-314 on tiny shapes."""

    xs = [[Fraction(float(v)) for v in row] for row in x.float().tolist()]
    gu = [[Fraction(float(v)) for v in row] for row in w_gate_up.float().tolist()]
    dn = [[Fraction(float(v)) for v in row] for row in w_down.float().tolist()]
    intermediate = len(dn[0])
    activated = []
    for row in xs:
        h_row = []
        for j in range(intermediate):
            gate = _bf16_round_fraction(sum(a * b for a, b in zip(row, gu[2 * j])))
            up = _bf16_round_fraction(sum(a * b for a, b in zip(row, gu[2 * j + 1])))
            g32 = np.float32(gate)
            silu = np.float32(g32 / (np.float32(1) + np.exp(-g32, dtype=np.float32)))
            h_row.append(_bf16_round_float(float(np.float32(silu * np.float32(up)))))
        activated.append(h_row)
    out = []
    for h_row in activated:
        out.append([_bf16_round_fraction(sum(Fraction(h) * w for h, w in zip(h_row, dn_row))) for dn_row in dn])
    return activated, out


def test_dense_partial_matches_exact_brute_force_on_reference_test_shape():
    # tests/suites/integration/runtime/ffnagent/test_operators.py:18-20 shape (4 x 16 x 8) with
    # the deterministic qualification weights (qualification.py:317-336).
    x = o.generate_hidden_states(4, 16, 17)
    w_gate_up, w_down = o.dense_layer_weights(hidden_size=16, intermediate_size=8)
    activated, out = _fraction_dense(x, w_gate_up, w_down)
    reference = o.dense_partial_reference(x, w_gate_up, w_down)
    assert reference.float().tolist() == out
    c_out, c_activated = c_oracle.dense_partial(x, w_gate_up, w_down)
    assert c_activated.float().tolist() == activated
    assert torch.equal(c_out.view(torch.int16), reference.view(torch.int16))


def _f16_round_float(value: float) -> float:
    """Round-to-nearest-even to IEEE binary16 (11 significant bits, subnormal spacing 2^-24)."""

    if value == 0 or not math.isfinite(value):
        return value
    _, exponent = math.frexp(value)
    quantum = Fraction(2) ** max(exponent - 11, -24)
    return float(_round_half_even(Fraction(value) / quantum) * quantum)


def test_fp16_payload_stages_match_exact_brute_force():
    # The fp16 payload (is_supported_payload_dtype, ffn.hpp:83-85) through the same Dense body
    # (qualification.py:290-314): exact rational projections rounded through fp32 to binary16,
    # fp32 SiLU*up rounded to binary16, exact down projection rounded to binary16.  The
    # brute force rounds with its own binary16 rule, so a bf16 rounding point left in the
    # oracle (8 significant bits instead of 11) fails here.
    x = o.generate_hidden_states(4, 16, 17).half()
    w_gate_up, w_down = (w.half() for w in o.dense_layer_weights(hidden_size=16, intermediate_size=8))
    xs = [[Fraction(float(v)) for v in row] for row in x.float().tolist()]
    gu = [[Fraction(float(v)) for v in row] for row in w_gate_up.float().tolist()]
    dn = [[Fraction(float(v)) for v in row] for row in w_down.float().tolist()]

    def to_f16(value: Fraction) -> float:
        return _f16_round_float(struct.unpack("f", struct.pack("f", float(value)))[0])

    expected = []
    for row in xs:
        activated = []
        for j in range(8):
            gate = np.float32(to_f16(sum(a * b for a, b in zip(row, gu[2 * j]))))
            up = np.float32(to_f16(sum(a * b for a, b in zip(row, gu[2 * j + 1]))))
            silu = np.float32(gate / (np.float32(1) + np.exp(-gate, dtype=np.float32)))
            activated.append(Fraction(_f16_round_float(float(np.float32(silu * up)))))
        expected.append([to_f16(sum(h * w for h, w in zip(activated, dn_row))) for dn_row in dn])
    reference = o.dense_partial_reference(x, w_gate_up, w_down)
    assert reference.dtype is torch.float16
    assert reference.float().tolist() == expected
    assert not torch.equal(reference.float(), o.dense_partial_reference(x.bfloat16(), w_gate_up.bfloat16(),
                                                                        w_down.bfloat16()).float())


def test_fp16_rmsnorm_gather_scatter_keep_the_payload_dtype():
    x = o.generate_hidden_states(8, 256, 21).half()
    weight = (1 + 0.1 * torch.randn(256, generator=torch.Generator().manual_seed(22))).half()
    result = o.rmsnorm(x, weight, 1e-6)
    assert result.dtype is torch.float16
    x64 = x.double()
    brute = (x64 / torch.sqrt((x64 * x64).mean(-1, keepdim=True) + 1e-6) * weight.double()).tolist()
    rounded = torch.tensor([[_f16_round_float(v) for v in row] for row in brute], dtype=torch.float64)
    ulp = torch.pow(2.0, torch.floor(torch.log2(rounded.abs().clamp_min(2.0**-14))) - 10)
    assert bool(((result.double() - rounded).abs() <= ulp).all())
    # gather / scatter move raw binary16 patterns, NaN payloads included
    pool = x.clone()
    pool.view(torch.int16)[3, :4] = torch.tensor([0x7E00, 0x7C01, -1, 0x0001], dtype=torch.int16)
    slots = np.array([3, 0, 6])
    gathered = o.gather(pool, slots)
    assert gathered.dtype is torch.float16
    assert torch.equal(gathered.view(torch.int16), pool[slots].view(torch.int16))
    scattered = o.scatter(pool, slots, gathered.flip(0).contiguous())
    assert scattered.dtype is torch.float16
    assert torch.equal(scattered[[6, 0, 3]].view(torch.int16), pool[slots].view(torch.int16))
    with pytest.raises(ValueError):
        o.scatter(pool, slots, gathered.bfloat16())


def test_dense_partial_matches_c_restatement_at_scale():
    x = o.generate_hidden_states(16, 256, 17)
    w_gate_up, w_down, _ = o.generate_layer(256, 384, 18)
    reference = o.dense_partial_reference(x, w_gate_up, w_down)
    c_out, _ = c_oracle.dense_partial(x, w_gate_up, w_down)
    assert torch.equal(c_out.view(torch.int16), reference.view(torch.int16))


def test_dense_invariants_catch_plausible_mistakes():
    x = o.generate_hidden_states(6, 32, 17)
    w_gate_up, w_down, _ = o.generate_layer(32, 16, 18)
    reference = o.dense_partial_reference(x, w_gate_up, w_down)
    # zero weights -> zero output (Control Capture Probes, weights.py:265-286)
    assert torch.equal(
        o.dense_partial_reference(x, torch.zeros_like(w_gate_up), w_down).float(), torch.zeros(6, 32)
    )
    # row independence: each row alone gives the same result
    for row in range(6):
        alone = o.dense_partial_reference(x[row : row + 1], w_gate_up, w_down)
        assert torch.equal(alone.view(torch.int16), reference[row : row + 1].view(torch.int16))
    # swapped Gate/Up (CONCATENATED vs INTERLEAVED confusion) changes the result
    swapped = o.interleave_gate_up(w_gate_up[1::2], w_gate_up[0::2])
    assert not torch.equal(o.dense_partial_reference(x, swapped, w_down), reference)
    # the down projection is linear in h: doubling w_down doubles the (exactly representable) output
    doubled = o.dense_partial_reference(x, w_gate_up, (w_down.float() * 2).to(torch.bfloat16))
    assert torch.equal(doubled.float(), reference.float() * 2)
    # silu closed forms
    assert float(o.silu(torch.tensor([0.0]))) == 0.0
    assert float(o.silu(torch.tensor([30.0]))) == pytest.approx(30.0)
    assert float(o.silu(torch.tensor([-30.0]))) == pytest.approx(0.0, abs=1e-10)


def test_gated_silu_transform_matches_c_restatement():
    generator = torch.Generator().manual_seed(3)
    gate = (torch.randn(4096, generator=generator) * 6).to(torch.bfloat16)
    up = (torch.randn(4096, generator=generator) * 6).to(torch.bfloat16)
    lib = c_oracle.library()
    for alpha, limit, offset in ((1.0, None, 0.0), (1.3, 4.0, -0.5)):
        ours = o.gated_silu(gate, up, alpha=alpha, limit=limit, up_offset=offset)
        theirs = np.array(
            [lib.xpo_gated_silu(int(g), int(u), alpha, limit or 0.0, offset)
             for g, u in zip(o.bf16_bits(gate), o.bf16_bits(up))],
            dtype=np.uint16,
        )
        mismatch = np.count_nonzero(o.bf16_bits(ours) != theirs)
        assert mismatch <= 4096 // 1000  # fp32 exp implementations may differ by an ulp


def test_tp_partials_sum_to_the_full_layer():
    # qualification.py:267-287: ordered fp32 sum of true-TP partials
    x = o.generate_hidden_states(3, 16, 17)
    shards = [o.dense_layer_weights(hidden_size=16, intermediate_size=8, tp_size=2, tp_rank=r) for r in range(2)]
    summed = o.dense_reference_sum(x, shards)
    manual = (o.dense_partial_reference(x, *shards[0]).float() + o.dense_partial_reference(x, *shards[1]).float())
    assert torch.equal(summed.float(), manual.to(torch.bfloat16).float())


def _bf16(values) -> torch.Tensor:
    return torch.tensor(values, dtype=torch.float32).to(torch.bfloat16)


def test_ordered_partial_sum_closed_forms():
    # delivery.cu:74-83: fp32 fold from +0 in PE order, one final bf16 cast.
    big = float(2**24)
    # (2^24 + 1) rounds to 2^24 in fp32, so the fold in order gives 0 and the reverse 1.
    assert torch.equal(o.ordered_partial_sum([_bf16([big]), _bf16([1.0]), _bf16([-big])]).float(), torch.tensor([0.0]))
    assert torch.equal(o.ordered_partial_sum([_bf16([-big]), _bf16([1.0]), _bf16([big])]).float(), torch.tensor([1.0]))
    # One rounding at the end: 1 + 2^-8 + 2^-8 = 1 + 2^-7 exactly (bf16 after every add
    # would round each 1 + 2^-8 tie back to 1).
    tiny = 2.0**-8
    assert o.ordered_partial_sum([_bf16([1.0]), _bf16([tiny]), _bf16([tiny])]).item() == 1.0 + 2.0**-7
    # A single partial is the identity, except that -0 becomes +0 (0.0 + -0.0).
    single = _bf16([-0.0, 3.5, -7.25, float("inf")])
    folded = o.ordered_partial_sum([single])
    assert o.bf16_bits(folded).tolist() == [0x0000] + o.bf16_bits(single).tolist()[1:]


def test_ordered_partial_sum_is_the_tp_layer_reference():
    # qualification.py:267-287: dense_reference sums the ordered partials the same way.
    x = o.generate_hidden_states(3, 16, 17)
    shards = [o.dense_layer_weights(hidden_size=16, intermediate_size=8, tp_size=4, tp_rank=r) for r in range(4)]
    partials = [o.dense_partial_reference(x, *shard) for shard in shards]
    assert torch.equal(o.ordered_partial_sum(partials), o.dense_reference_sum(x, shards))


def test_deterministic_weights_are_exact_bf16():
    gate, up, down = o.dense_full_weights(hidden_size=16, intermediate_size=8)
    for tensor, offset in ((gate, 3), (up, 11), (down, 19)):
        data = torch.arange(tensor.numel(), dtype=torch.float64)
        expected = (((data + offset) % 29) - 14) / 64
        assert torch.equal(tensor.double().flatten(), expected)


# --------------------------------------------------------------- capacities / workspace
def test_capacity_buckets_match_reference_known_answers():
    # tests/suites/unit/runtime/ffnagent/test_execution.py:18-24
    assert o.derive_payload_row_capacities(1) == (1,)
    assert o.derive_payload_row_capacities(5) == (1, 2, 4, 5)
    assert o.derive_payload_row_capacities(8) == (1, 2, 4, 8)
    with pytest.raises(ValueError, match="positive"):
        o.derive_payload_row_capacities(0)
    assert o.select_capacity((1, 2, 4, 5), 3) == 4
    assert o.select_capacity((1, 2, 4, 5), 5) == 5
    assert o.select_capacity((1, 2, 4, 5), 6) is None


def test_workspace_offsets_match_reference_known_answers():
    # test_execution.py:26-60: gated CONCATENATED 4x16x8 bf16 -> 192 bytes, activated at +128.
    offsets, total = o.workspace_offsets([4 * 16 * 2, 4 * 8 * 2, 0, 0])
    assert total == 192 and offsets[1] == 128
    offsets, total = o.workspace_offsets([3, 5])
    assert offsets == (0, 16) and total == 21


# --------------------------------------------------------------- golden fixtures
def test_golden_dense_fixture_reproduces():
    golden = np.load(GOLDEN_DIR / "dense_4x16x8.npz")
    x = o.bf16_from_bits(golden["x"])
    w_gate_up = o.bf16_from_bits(golden["w_gate_up"])
    w_down = o.bf16_from_bits(golden["w_down"])
    assert np.array_equal(o.bf16_bits(o.dense_partial_reference(x, w_gate_up, w_down)), golden["out"])
    gate_up, down = o.dense_layer_weights(hidden_size=16, intermediate_size=8)
    assert np.array_equal(o.bf16_bits(gate_up), golden["w_gate_up"])
    assert np.array_equal(o.bf16_bits(down), golden["w_down"])


def test_golden_mailbox_fixture_reproduces():
    golden = np.load(GOLDEN_DIR / "mailbox_32x128.npz")
    pool = o.bf16_from_bits(golden["pool"])
    new_pool, normalized, rows = o.mailbox_step(
        pool,
        golden["slots"],
        o.bf16_from_bits(golden["w_gate_up"]),
        o.bf16_from_bits(golden["w_down"]),
        norm_weight=o.bf16_from_bits(golden["norm_weight"]),
        eps=float(golden["eps"][0]),
    )
    assert np.array_equal(o.bf16_bits(normalized), golden["normalized"])
    assert np.array_equal(o.bf16_bits(rows), golden["ffn_rows"])
    assert np.array_equal(o.bf16_bits(new_pool), golden["new_pool"])
    c_rows, _ = c_oracle.dense_partial(normalized, o.bf16_from_bits(golden["w_gate_up"]), o.bf16_from_bits(golden["w_down"]))
    assert np.array_equal(o.bf16_bits(c_rows), golden["ffn_rows"])


# --------------------------------------------------------------------------- #
# Activations and the general projection (operators/activation.py, linear.py)
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_relu_bits_match_torch_except_where_the_reference_rule_differs(dtype):
    # activation.py:19-27: the pattern where v > 0 or v is NaN, +0 otherwise.  torch's CPU
    # relu agrees on every other pattern; it keeps -0 and canonicalises NaNs, where the
    # reference's rule gives +0 and keeps the payload (what its all-pattern test pins on CUDA).
    values = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(dtype)
    got = o.relu_bits(values).view(torch.int16)
    f = values.float()
    ordinary = (f == f) & ~((f == 0) & (values.view(torch.int16) < 0))
    assert torch.equal(got[ordinary], values.relu().view(torch.int16)[ordinary])
    nan = f != f
    assert int(nan.sum()) > 0 and torch.equal(got[nan], values.view(torch.int16)[nan])
    negative_zero = torch.tensor([-0.0], dtype=dtype)
    assert int(o.relu_bits(negative_zero).view(torch.int16).item()) == 0


def test_activation_functions_match_torch_library_routines():
    x = torch.linspace(-12, 12, 4801, dtype=torch.float32)
    torch.testing.assert_close(o.activation_function(x, "silu"), torch.nn.functional.silu(x), rtol=2e-6, atol=1e-7)
    torch.testing.assert_close(o.activation_function(x, "silu", alpha=1.702), x * torch.sigmoid(1.702 * x),
                               rtol=2e-6, atol=1e-7)
    for approximate in ("none", "tanh"):
        torch.testing.assert_close(o.activation_function(x, "gelu", approximate=approximate),
                                   torch.nn.functional.gelu(x, approximate=approximate), rtol=2e-6, atol=1e-6)
    # a wrong slope or the other GELU form fails the same check
    assert not torch.allclose(o.activation_function(x, "silu", alpha=1.3), torch.nn.functional.silu(x), atol=1e-3)
    assert not torch.allclose(o.activation_function(x, "gelu", approximate="tanh"),
                              torch.nn.functional.gelu(x), rtol=0, atol=1e-6)


def test_gated_activation_clip_and_offset_closed_forms():
    gate = torch.tensor([10.0, -10.0, 2.0, 0.5])
    up = torch.tensor([9.0, -9.0, 1.0, -0.25])
    got = o.gated_activation(gate, up, function="relu", limit=4.0, up_offset=-0.5)
    # gate clipped above only (10 -> 4, -10 stays), up clamped to [-4, 4], then + offset
    expected = torch.tensor([4.0 * (4.0 - 0.5), 0.0 * (-4.0 - 0.5), 2.0 * (1.0 - 0.5), 0.5 * (-0.25 - 0.5)])
    assert torch.equal(got, expected)
    # no limit: identity transform
    assert torch.equal(o.gated_activation(gate, up, function="relu"), torch.relu(gate) * up)


def test_standalone_activation_orders_agree_on_permuted_inputs():
    g = torch.Generator().manual_seed(3)
    gate = torch.randn((6, 40), generator=g).to(torch.bfloat16)
    up = torch.randn((6, 40), generator=g).to(torch.bfloat16)
    interleaved = torch.stack((gate, up), dim=2).reshape(6, 80)
    concatenated = torch.cat((gate, up), dim=1)
    kwargs = dict(width=40, function="silu", gated=True, alpha=1.3, limit=4.0, up_offset=-0.5)
    a = o.standalone_activation(interleaved, order="interleaved", **kwargs)
    b = o.standalone_activation(concatenated, order="concatenated", **kwargs)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    # reading the other order's layout gives a different result
    c = o.standalone_activation(interleaved, order="concatenated", **kwargs)
    assert not torch.equal(a.view(torch.int16), c.view(torch.int16))


def test_projection_reference_adds_the_bias_before_the_rounding_point():
    # x . w = 1 + 2^-8 exactly (halfway between bf16 1 and 1 + 2^-7: rounds to 1, even);
    # a bias of 2^-9 lifts it past the halfway point, so the result must be 1 + 2^-7.  Adding the
    # bias after rounding would give 1 + 2^-9 -> 1.
    x = torch.tensor([[1.0, 2.0**-8]], dtype=torch.bfloat16)
    w = torch.tensor([[1.0, 1.0]], dtype=torch.bfloat16)
    assert o.projection_reference(x, w).float().item() == 1.0
    bias = torch.tensor([2.0**-9])
    assert o.projection_reference(x, w, bias).float().item() == 1.0 + 2.0**-7
    # gated epilogue: the projection is rounded before the activation (relu of the rounded sum)
    w2 = torch.tensor([[1.0, 1.0], [1.0, 0.0]], dtype=torch.bfloat16)  # gate row, up row
    out = o.projection_reference(x, w2, function="relu", gated=True)
    assert out.float().item() == 1.0 * 1.0  # gate rounds to 1 (not 1 + 2^-8), up = 1
