"""The GPU parity bars of tests/parity.py, exercised on the CPU.

A bar is only worth something if a correct fp32-accumulating implementation passes it
and plausible mistakes fail it.  Here the "implementation" is computed on the CPU:
an fp32 torch matmul with the reference's rounding points must pass every bar, and the
same computation with one planted mistake (a transposed weight operand, Gate/Up rows
swapped, the up factor dropped, the stage rounding of gate/up skipped, the output
rounded once more, a wrong sign, a row reading its neighbour's slot) must fail.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ffn_oracle as o
from parity import (
    assert_activated_within_bounds,
    assert_bitwise_equal,
    assert_ffn_parity,
    assert_projection_within_bounds,
)

ROWS, HIDDEN, INTERMEDIATE = 24, 256, 96


@pytest.fixture(scope="module")
def case():
    x = o.generate_hidden_states(ROWS, HIDDEN, 17)
    w_gate_up, w_down, _ = o.generate_layer(HIDDEN, INTERMEDIATE, 18)
    return x, w_gate_up, w_down


def _fp32_projection(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return (x.float() @ w.float().t()).to(torch.bfloat16)


def _fp32_activated(x, w_gate_up, *, round_stage=True, drop_up=False):
    projected = x.float() @ w_gate_up.float().t()
    gate, up = projected[:, 0::2], projected[:, 1::2]
    if round_stage:
        gate, up = gate.to(torch.bfloat16).float(), up.to(torch.bfloat16).float()
    if drop_up:
        up = torch.ones_like(up)
    return (gate / (1.0 + torch.exp(-gate)) * up).to(torch.bfloat16)


def test_fp32_implementation_passes_every_bar(case):
    x, w_gate_up, w_down = case
    activated = _fp32_activated(x, w_gate_up)
    assert_activated_within_bounds(activated, x, w_gate_up)
    out = _fp32_projection(activated, w_down)
    assert_projection_within_bounds(out, activated, w_down)
    stage = o.dense_partial_reference(x, w_gate_up, w_down)
    assert_ffn_parity(out, stage, o.dense_fp32(x, w_gate_up, w_down))


def test_projection_bar_catches_a_transposed_operand(case):
    _, _, w_down = case
    h = o.generate_hidden_states(ROWS, INTERMEDIATE, 29)
    square = w_down[:INTERMEDIATE, :INTERMEDIATE]  # square so the transpose has the same shape
    with pytest.raises(AssertionError):
        assert_projection_within_bounds(_fp32_projection(h, square.t().contiguous()), h, square)


def test_projection_bar_catches_a_wrong_sign_and_an_extra_rounding(case):
    _, _, w_down = case
    h = o.generate_hidden_states(ROWS, INTERMEDIATE, 29)
    with pytest.raises(AssertionError):
        assert_projection_within_bounds(-_fp32_projection(h, w_down), h, w_down)
    # rounding the output through fp16 first (a double rounding) moves many elements
    coarse = (h.float() @ w_down.float().t()).to(torch.float16).to(torch.bfloat16)
    scaled = coarse * 1.0078125  # and one ulp-scale bias on top
    with pytest.raises(AssertionError):
        assert_projection_within_bounds(scaled, h, w_down)


@pytest.mark.parametrize("mistake", ["swapped", "drop_up", "no_stage_rounding"])
def test_activation_bar_catches_plausible_mistakes(case, mistake):
    x, w_gate_up, _ = case
    if mistake == "swapped":
        swapped = o.interleave_gate_up(w_gate_up[1::2], w_gate_up[0::2])
        wrong = _fp32_activated(x, swapped)
    elif mistake == "drop_up":
        wrong = _fp32_activated(x, w_gate_up, drop_up=True)
    else:
        wrong = _fp32_activated(x, w_gate_up, round_stage=False)
    with pytest.raises(AssertionError):
        assert_activated_within_bounds(wrong, x, w_gate_up)


def test_ffn_bar_catches_a_layer_with_the_wrong_down_weights(case):
    x, w_gate_up, w_down = case
    stage = o.dense_partial_reference(x, w_gate_up, w_down)
    wrong = o.dense_partial_reference(x, w_gate_up, torch.roll(w_down, shifts=1, dims=1))
    with pytest.raises(AssertionError):
        assert_ffn_parity(wrong, stage, o.dense_fp32(x, w_gate_up, w_down))


def test_bitwise_bar_catches_a_row_read_from_the_neighbouring_slot():
    pool = o.generate_hidden_states(64, 128, 17)
    slots = o.generate_slots(64, 16, 19)
    expected = o.gather(pool, slots)
    shifted = slots.copy()
    shifted[3] = (shifted[3] + 1) % 64
    with pytest.raises(AssertionError):
        assert_bitwise_equal(o.gather(pool, shifted), expected)
