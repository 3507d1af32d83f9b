"""Generate the small golden fixtures under tests/golden/ (run from the repo root).

The reference keeps no stored tensor fixtures for this path (every reference
test computes its expectation in torch), so these vectors come from this
repo's oracle after the oracle has been pinned (tests/test_oracle.py): the C
restatement, exact rational brute force and closed forms.  They freeze the
oracle's outputs so a later change to either side is caught.

* ``dense_4x16x8.npz``: the reference operator-test shape
  (tests/suites/integration/runtime/ffnagent/test_operators.py:18-20) with the
  deterministic qualification weights (qualification.py:317-336) and seeded
  N(0,1) bf16 rows (seed 17).
* ``mailbox_32x128.npz``: a 32-slot mailbox of width 128, 8 seeded slots,
  RMSNorm weight 1+N(0,0.1), Dense I = 256 with N(0, 0.02) weights: the new
  pool, the normalised batch and the FFN rows.

bf16 tensors are stored as uint16 bit patterns.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import ffn_oracle as o  # noqa: E402


def dense_fixture() -> dict[str, np.ndarray]:
    x = o.generate_hidden_states(4, 16, 17)
    w_gate_up, w_down = o.dense_layer_weights(hidden_size=16, intermediate_size=8)
    out = o.dense_partial_reference(x, w_gate_up, w_down)
    projected = x.double() @ w_gate_up.double().t()
    activated = o.gated_silu(projected[:, 0::2].bfloat16(), projected[:, 1::2].bfloat16())
    return {
        "x": o.bf16_bits(x),
        "w_gate_up": o.bf16_bits(w_gate_up),
        "w_down": o.bf16_bits(w_down),
        "activated": o.bf16_bits(activated),
        "out": o.bf16_bits(out),
    }


def mailbox_fixture() -> dict[str, np.ndarray]:
    pool = o.generate_hidden_states(32, 128, 17)
    w_gate_up, w_down, norm_weight = o.generate_layer(128, 256, 18)
    slots = o.generate_slots(32, 8, 19)
    new_pool, normalized, ffn_rows = o.mailbox_step(pool, slots, w_gate_up, w_down, norm_weight=norm_weight)
    return {
        "pool": o.bf16_bits(pool),
        "w_gate_up": o.bf16_bits(w_gate_up),
        "w_down": o.bf16_bits(w_down),
        "norm_weight": o.bf16_bits(norm_weight),
        "slots": slots,
        "eps": np.array([1e-6], dtype=np.float32),
        "normalized": o.bf16_bits(normalized),
        "ffn_rows": o.bf16_bits(ffn_rows),
        "new_pool": o.bf16_bits(new_pool),
    }


def main() -> None:
    np.savez_compressed(HERE / "dense_4x16x8.npz", **dense_fixture())
    np.savez_compressed(HERE / "mailbox_32x128.npz", **mailbox_fixture())
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
