"""GPU parity of the Transport kernels: byte copy, gather (+RMSNorm), scatter.

Bar: bit-exact for copies, gathers and scatters; RMSNorm within one bf16 ulp
of the fp32 oracle with >= 99 % of elements bit-identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from crosspool_amd import _native, dense
from oracle import ffn_oracle as o
from parity import assert_bitwise_equal, assert_within_ulps, slots_tensor, to_device

pytestmark = pytest.mark.gpu


# --------------------------------------------------------------- byte copy
# The reference's cooperative-copy cases (tests/suites/cext/utils/cooperative_test.cu:77-111):
# (destination offset, source offset, bytes) over a 256-byte allocation.
@pytest.mark.parametrize("dst_offset,src_offset,count", [(32, 16, 128), (7, 3, 128), (32, 16, 127), (0, 0, 256)])
def test_copy_bytes_matches_cooperative_copy_cases(device, dst_offset, src_offset, count):
    allocation = 256
    source = torch.tensor([(i * 17 + 3) % 251 for i in range(allocation)], dtype=torch.uint8)
    destination = torch.full((allocation,), 0xA5, dtype=torch.uint8)
    expected = destination.numpy().copy()
    o.copy_bytes(expected[dst_offset : dst_offset + count], source.numpy()[src_offset : src_offset + count])
    src_gpu, dst_gpu = source.to(device), destination.to(device)
    dense.copy_bytes(dst_gpu[dst_offset : dst_offset + count], src_gpu[src_offset : src_offset + count])
    torch.cuda.synchronize()
    assert np.array_equal(dst_gpu.cpu().numpy(), expected)
    assert torch.equal(src_gpu.cpu(), source)


def test_copy_bytes_zero_length_with_null_pointers(device):
    assert _native.library().xp_copy_bytes(None, None, 0, None) == 0


def test_copy_bytes_large_aligned(device):
    source = torch.randint(0, 256, (33 * 1024 * 1024 + 48,), dtype=torch.uint8, device=device)
    destination = torch.zeros_like(source)
    dense.copy_bytes(destination, source)
    torch.cuda.synchronize()
    assert torch.equal(destination, source)


# --------------------------------------------------------------- gather
@pytest.mark.parametrize("hidden", [8, 128, 1024, 2048, 2560, 4096, 5120, 8200])
@pytest.mark.parametrize("rows", [1, 5, 64, 257])
def test_plain_gather_is_bit_exact(device, hidden, rows):
    pool_rows = max(rows, 300)
    pool = o.generate_hidden_states(pool_rows, hidden, 17)
    slots = o.generate_slots(pool_rows, rows, 19)
    out = dense.gather_rmsnorm(to_device(pool, device), slots_tensor(slots, device))
    torch.cuda.synchronize()
    assert_bitwise_equal(out, o.gather(pool, slots))


def test_identity_slots_reproduce_the_reference_prefix_copy(device):
    # src/cext/transport/instance.cu:83-84 copies bytes [0, T*H*2) of the caller's rows.
    pool = o.generate_hidden_states(64, 4096, 17)
    rows = 33
    out = dense.gather_rmsnorm(to_device(pool, device), torch.arange(rows, dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    assert out.cpu().view(torch.uint8).numpy().tobytes() == pool[:rows].view(torch.uint8).numpy().tobytes()


@pytest.mark.parametrize("hidden", [1024, 2048, 2560, 4096, 5120])
def test_gather_rmsnorm_matches_oracle(device, hidden):
    pool = o.generate_hidden_states(512, hidden, 17)
    _, _, norm_weight = o.generate_layer(hidden, 8, 18)
    slots = o.generate_slots(512, 200, 19)
    out = dense.gather_rmsnorm(
        to_device(pool, device), slots_tensor(slots, device), norm_weight=to_device(norm_weight, device), eps=1e-6
    )
    torch.cuda.synchronize()
    expected = o.rmsnorm(o.gather(pool, slots), norm_weight, 1e-6)
    assert_within_ulps(out, expected, ulps=1.0, exact_fraction=0.99)


def test_gather_rmsnorm_eps_dominated_and_zero_rows(device):
    hidden = 1024
    pool = torch.zeros((4, hidden), dtype=torch.bfloat16)
    pool[1] = 1e-3
    pool[2] = -3.0
    pool[3] = o.generate_hidden_states(1, hidden, 5)[0]
    weight = torch.ones(hidden, dtype=torch.bfloat16)
    slots = np.array([0, 1, 2, 3], dtype=np.int32)
    out = dense.gather_rmsnorm(
        to_device(pool, device), slots_tensor(slots, device), norm_weight=to_device(weight, device), eps=1e-6
    ).cpu()
    assert torch.equal(out[0].float(), torch.zeros(hidden))  # 0 * 1/sqrt(eps)
    # Constant rows: x / sqrt(x^2 + eps), with x the bf16 value of 1e-3 (eps is not negligible).
    x = float(pool[1, 0].float())
    assert_within_ulps(out[1], torch.full((hidden,), x / (x * x + 1e-6) ** 0.5, dtype=torch.bfloat16))
    assert_within_ulps(out[2], torch.full((hidden,), -1.0, dtype=torch.bfloat16))
    assert_within_ulps(out[3:], o.rmsnorm(pool[3:], weight), exact_fraction=0.99)


def test_gather_out_of_range_slot_poisons_row_and_raises_fault(device):
    pool = o.generate_hidden_states(16, 1024, 17)
    slots = np.array([3, 16, 5, -1], dtype=np.int32)
    fault = torch.zeros(1, dtype=torch.int32, device=device)
    out = dense.gather_rmsnorm(to_device(pool, device), slots_tensor(slots, device), fault_word=fault).cpu()
    assert int(fault.item()) == _native.XP_FAULT_SLOT_OUT_OF_RANGE
    assert torch.isnan(out[1].float()).all() and torch.isnan(out[3].float()).all()
    assert_bitwise_equal(out[0::2], o.gather(pool, np.array([3, 5])))


def test_zero_rows_is_a_no_op(device):
    pool = torch.zeros((4, 64), dtype=torch.bfloat16, device=device)
    out = dense.gather_rmsnorm(pool, torch.zeros(0, dtype=torch.int32, device=device))
    assert out.shape == (0, 64)


def test_gather_rejects_rows_that_are_not_16_byte_multiples(device):
    pool = torch.zeros((4, 12), dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        dense.gather_rmsnorm(pool, torch.zeros(2, dtype=torch.int32, device=device))


# --------------------------------------------------------------- scatter
@pytest.mark.parametrize("hidden,rows", [(1024, 64), (4096, 1), (4096, 300), (2560, 17)])
def test_scatter_is_bit_exact(device, hidden, rows):
    pool = o.generate_hidden_states(512, hidden, 17)
    values = o.generate_hidden_states(rows, hidden, 23)
    slots = o.generate_slots(512, rows, 19)
    pool_gpu = to_device(pool, device)
    dense.scatter(to_device(values, device), slots_tensor(slots, device), pool_gpu)
    torch.cuda.synchronize()
    assert_bitwise_equal(pool_gpu, o.scatter(pool, slots, values))


def test_scatter_skips_out_of_range_slots(device):
    pool = o.generate_hidden_states(8, 64, 17)
    values = o.generate_hidden_states(2, 64, 23)
    fault = torch.zeros(1, dtype=torch.int32, device=device)
    pool_gpu = to_device(pool, device)
    dense.scatter(to_device(values, device), slots_tensor(np.array([2, 8]), device), pool_gpu, fault_word=fault)
    torch.cuda.synchronize()
    assert int(fault.item()) == _native.XP_FAULT_SLOT_OUT_OF_RANGE
    assert_bitwise_equal(pool_gpu, o.scatter(pool, np.array([2]), values[:1]))
