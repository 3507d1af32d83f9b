"""GPU parity of the fixed-order TP partial reduction (xp_reduce_partials).

Bit-exact against the oracle's fold (delivery.cu:74-83 order: fp32 from +0, partials in
rank order, one bf16 cast), at the Qwen3-32B 1/8-shard partial shape (config 5) and on
the closed-form cases where the order or the single final rounding decides the result.
"""

from __future__ import annotations

import pytest
import torch

from crosspool_amd import _native
from crosspool_amd.delivery import reduce_tp_partials
from oracle import ffn_oracle as o
from parity import assert_bitwise_equal

pytestmark = pytest.mark.gpu


def _partials(count: int, shape: tuple[int, ...], seed: int) -> list[torch.Tensor]:
    generator = torch.Generator().manual_seed(seed)
    return [(torch.randn(shape, generator=generator) * (1 + k)).to(torch.bfloat16) for k in range(count)]


@pytest.mark.parametrize(
    ("count", "shape"),
    # The last case (4 x 84 MB) is larger than the last-level cache, so the kernel takes its
    # nontemporal loads and stores.
    [(1, (8,)), (2, (3, 1024)), (3, (17, 2560)), (8, (512, 5120)), (16, (64, 4096)), (4, (8192, 5120))],
)
def test_reduction_matches_the_ordered_fold(device, count, shape):
    print(f"reduce partials count={count} shape={shape}", flush=True)
    partials = _partials(count, shape, 40 + count)
    out = reduce_tp_partials([p.to(device) for p in partials])
    torch.cuda.synchronize()
    assert_bitwise_equal(out.cpu(), o.ordered_partial_sum(partials))


def test_reduction_order_and_single_rounding(device):
    big, tiny = float(2**24), 2.0**-8
    rows = [[big, 1.0, -0.0, 1.0], [1.0, -big, -0.0, tiny], [-big, big, -0.0, tiny]]
    partials = [torch.tensor(row * 2, dtype=torch.float32).to(torch.bfloat16) for row in rows]
    # Partial order: 2^24 + 1 rounds to 2^24 in fp32, so column 0 folds to 0 and column 1
    # (1 - 2^24 exact, + 2^24) to 1; -0 + -0 + -0 from +0 is +0; 1 + 2^-8 + 2^-8 is rounded
    # once (a bf16 rounding after each add would give 1).
    out = reduce_tp_partials([p.to(device) for p in partials]).cpu()
    assert_bitwise_equal(out, o.ordered_partial_sum(partials))
    assert out[:4].float().tolist() == [0.0, 1.0, 0.0, 1.0 + 2.0**-7]
    assert o.bf16_bits(out)[2] == 0


def test_output_may_alias_a_partial(device):
    partials = _partials(4, (33, 512), 7)
    on_device = [p.to(device) for p in partials]
    out = reduce_tp_partials(on_device, out=on_device[2])
    assert out.data_ptr() == on_device[2].data_ptr()
    assert_bitwise_equal(out.cpu(), o.ordered_partial_sum(partials))


def test_reduction_rejects_bad_arguments(device):
    good = torch.zeros(64, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="between 1 and 16"):
        reduce_tp_partials([good] * 17)
    with pytest.raises(ValueError, match="one shape"):
        reduce_tp_partials([good, torch.zeros(72, dtype=torch.bfloat16, device=device)])
    unaligned = torch.zeros(72, dtype=torch.bfloat16, device=device)[1:65]
    with pytest.raises(_native.NativeError, match="16-byte aligned"):
        reduce_tp_partials([good, unaligned])
    with pytest.raises(_native.NativeError, match="multiple of 8"):
        reduce_tp_partials([torch.zeros(12, dtype=torch.bfloat16, device=device)])
