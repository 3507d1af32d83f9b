"""xp_dense_step_static (the Dense step over the library's static device scratch) against
xp_dense_step (the same kernels over a caller workspace).

Both run the same kernel chain with the same arguments apart from the workspace address, and
every kernel is deterministic, so the mailboxes must agree bit for bit.  Two calls in a row on
the static scratch, the second with fewer rows, check that nothing of the first call's contents
leaks into the second; a step needing more than the scratch holds is refused before any
device work.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from crosspool_amd import _native
from oracle import ffn_oracle as o
from parity import assert_bitwise_equal, slots_tensor, to_device

pytestmark = pytest.mark.gpu

STATIC_SCRATCH_BYTES = 64 << 20


def _p(tensor):
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def _step(static, pool, slots, rows, w_gate_up, w_down, norm, fault, workspace=None):
    hidden, intermediate = w_down.shape
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if static:
        return _native.library().xp_dense_step_static(
            _p(pool), _p(pool), pool.shape[0], _p(slots), rows, hidden, intermediate, _p(w_gate_up), _p(w_down),
            _p(norm), 1e-6, _p(fault), stream,
        )
    return _native.library().xp_dense_step(
        _p(pool), _p(pool), pool.shape[0], _p(slots), rows, hidden, intermediate, _p(w_gate_up), _p(w_down),
        _p(norm), 1e-6, _p(workspace), workspace.numel(), _p(fault), stream,
    )


@pytest.mark.parametrize("hidden,intermediate,sizes", [
    (4096, 12288, (256, 16)),   # tile kernels with a split-K down, then the fused-gather stream kernel
    (1024, 3072, (300, 33)),    # tile kernels with split-K partials at both sizes
    (5120, 3200, (8, 1)),       # split kernels
])
def test_static_step_matches_workspace_step(device, hidden, intermediate, sizes):
    pool_rows = 1024
    w_gate_up, w_down, norm_weight = o.generate_layer(hidden, intermediate, 18)
    gu, dn, norm = to_device(w_gate_up, device), to_device(w_down, device), to_device(norm_weight, device)
    pool = o.generate_hidden_states(pool_rows, hidden, 17)
    fault = torch.zeros(1, dtype=torch.int32, device=device)
    static_pool = to_device(pool, device)
    reference_pool = to_device(pool, device)
    for call, rows in enumerate(sizes):
        assert _native.dense_workspace_bytes(rows, hidden, intermediate) <= STATIC_SCRATCH_BYTES
        print(f"case hidden={hidden} intermediate={intermediate} call={call} rows={rows}", flush=True)
        slots = slots_tensor(o.generate_slots(pool_rows, rows, 19 + call), device)
        workspace = torch.empty(_native.dense_workspace_bytes(rows, hidden, intermediate), dtype=torch.uint8,
                                device=device)
        assert _step(True, static_pool, slots, rows, gu, dn, norm, fault) == _native.XP_OK, _native.last_error()
        assert _step(False, reference_pool, slots, rows, gu, dn, norm, fault, workspace) == _native.XP_OK
        torch.cuda.synchronize()
        assert_bitwise_equal(static_pool.cpu(), reference_pool.cpu())
    assert int(fault.item()) == 0
    # Every slot touched by the two calls changed, the others did not.
    touched = np.union1d(o.generate_slots(pool_rows, sizes[0], 19), o.generate_slots(pool_rows, sizes[1], 20))
    untouched = np.setdiff1d(np.arange(pool_rows), touched)
    assert_bitwise_equal(static_pool.cpu()[untouched], pool[untouched])


def test_static_step_refuses_steps_past_the_scratch(device):
    hidden, intermediate, rows = 4096, 12288, 4096
    assert _native.dense_workspace_bytes(rows, hidden, intermediate) > STATIC_SCRATCH_BYTES
    pool = torch.zeros((rows, hidden), dtype=torch.bfloat16, device=device)
    gu = torch.zeros((2 * intermediate, hidden), dtype=torch.bfloat16, device=device)
    dn = torch.zeros((hidden, intermediate), dtype=torch.bfloat16, device=device)
    slots = torch.arange(rows, dtype=torch.int32, device=device)
    before = pool.clone()
    status = _step(True, pool, slots, rows, gu, dn, None, None)
    assert status == _native.XP_ERROR_CAPACITY
    assert "static scratch" in _native.last_error()
    torch.cuda.synchronize()
    assert_bitwise_equal(pool.cpu(), before.cpu())
