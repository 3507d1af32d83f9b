"""GPU parity at the sizes bench.py times: BASELINE config 3 (Qwen3-8B FFN layer) at 1024,
2048 and 4096 rows and config 5 (a Qwen3-32B tensor-parallel shard) at 512 and 8192 rows.

Each case runs one FfnAgent step (the Lane's template replay, the kernels the bench times)
and checks every stage on the GPU's own previous stage, read back from the Lane workspace:

* rows outside the slots are untouched, bit for bit;
* the gathered, RMS-normalised batch is within 1 bf16 ulp of the oracle's RMSNorm of the
  gathered rows (>= 99 % bit-identical);
* the activated intermediate lies in the rigorous fp32-accumulation intervals of the GPU's
  batch (tests/parity.py) on a row sample that covers every 256-row token tile: 37 rows per
  tile, 7 apart, so every row position of a 32-row MFMA block and every wave band of every
  tile shape; all columns, so every weight tile;
* the output rows lie in their intervals from the GPU's activated rows (same sample);
* every output row meets the FFN bar of tests/parity.py against the oracle's mailbox step
  (reference rounding points) and the pure-fp32 oracle; max-abs against fp32 is printed.

The kernels each case reaches are asserted by name (the chooser is a pure host function).
"""

from __future__ import annotations

from functools import lru_cache

import numpy as np
import pytest
import torch

from crosspool_amd import _native
from crosspool_amd.agent import FfnAgent
from crosspool_amd.weights import DenseFfnWeights
from oracle import ffn_oracle as o
from parity import (
    assert_activated_within_bounds,
    assert_bitwise_equal,
    assert_ffn_parity,
    assert_projection_within_bounds,
    assert_within_ulps,
    slots_tensor,
    to_device,
)

pytestmark = pytest.mark.gpu

QWEN3_8B = (4096, 12288)
QWEN3_32B_SHARD = (5120, 3200)

# (hidden, intermediate, rows, pool rows, normed, gate_up variant, down variant)
CASES = [
    pytest.param(*QWEN3_8B, 1024, 8192, True, "tile_gated_256x256+256x128_n8192", "tile_256x256_k4", id="config3-T1024"),
    pytest.param(*QWEN3_8B, 2048, 8192, True, "tile_gated_256x256", "tile_256x128", id="config3-T2048"),
    pytest.param(*QWEN3_8B, 4096, 8192, True, "tile_gated_256x256", "tile_256x256", id="config3-T4096"),
    pytest.param(*QWEN3_32B_SHARD, 512, 8192, False, "tile_gated_128x128", "tile_128x128", id="config5-T512"),
    pytest.param(*QWEN3_32B_SHARD, 8192, 8192, False, "tile_gated_256x256+64x128_n256", "tile_256x256+256x128_n1024",
                 id="config5-T8192"),
]


@lru_cache(maxsize=2)
def _layer(hidden: int, intermediate: int):
    return o.generate_layer(hidden, intermediate, 18)


@lru_cache(maxsize=2)
def _pool(pool_rows: int, hidden: int):
    return o.generate_hidden_states(pool_rows, hidden, 17)


def sample_rows(rows: int) -> np.ndarray:
    """37 rows 7 apart in every 256-row token tile (plus each tile's last row)."""

    picked = set()
    for tile in range(0, rows, 256):
        for offset in list(range(0, 256, 7)) + [255]:
            if tile + offset < rows:
                picked.add(tile + offset)
    return np.array(sorted(picked), dtype=np.int64)


def test_row_sample_covers_every_tile_position():
    rows = sample_rows(2048)
    for tile in range(8):
        in_tile = rows[(rows >= 256 * tile) & (rows < 256 * (tile + 1))] % 256
        assert set(in_tile % 32) == set(range(32))
        assert set(in_tile // 64) == {0, 1, 2, 3}


@pytest.mark.parametrize("hidden,intermediate,rows,pool_rows,normed,gate_up_variant,down_variant", CASES)
def test_headline_layer_stages(device, hidden, intermediate, rows, pool_rows, normed, gate_up_variant, down_variant):
    assert _native.gemm_variant(rows, 2 * intermediate, hidden, True) == gate_up_variant
    assert _native.gemm_variant(rows, hidden, intermediate, False) == down_variant
    w_gate_up, w_down, norm_weight = _layer(hidden, intermediate)
    if not normed:
        norm_weight = None
    pool = _pool(pool_rows, hidden)
    slots = o.generate_slots(pool_rows, rows, 19)
    print(f"case hidden={hidden} intermediate={intermediate} rows={rows} variants={gate_up_variant},{down_variant}",
          flush=True)
    with FfnAgent(device) as agent:
        agent.register_layer(
            instance_index=0, layer_ordinal=0,
            weights=DenseFfnWeights.from_tensors(to_device(w_gate_up, device), to_device(w_down, device)),
            norm_weight=None if norm_weight is None else to_device(norm_weight, device),
        )
        agent.materialize(maximum_row_capacity=rows)
        lane = agent.lanes[0]
        pool_gpu = to_device(pool, device)
        agent.execute(instance_index=0, layer_ordinal=0, pool=pool_gpu, slots=slots_tensor(slots, device))
        agent.check_health()
        batch_at, activated_at, _, _, _ = _native.dense_workspace_layout(rows, hidden, intermediate)
        workspace = lane.workspace.cpu()
        new_pool = pool_gpu.cpu()
    batch = workspace[batch_at:batch_at + rows * hidden * 2].view(torch.bfloat16).view(rows, hidden)
    activated = workspace[activated_at:activated_at + rows * intermediate * 2].view(torch.bfloat16)
    activated = activated.view(rows, intermediate)

    untouched = np.setdiff1d(np.arange(pool_rows), slots)
    assert_bitwise_equal(new_pool[untouched], pool[untouched])
    gathered = o.gather(pool, slots)
    if norm_weight is None:
        assert_bitwise_equal(batch, gathered)
    else:
        assert_within_ulps(batch, o.rmsnorm(gathered, norm_weight, 1e-6), ulps=1.0, exact_fraction=0.99)

    picked = torch.from_numpy(sample_rows(rows))
    output = o.gather(new_pool, slots)
    assert_activated_within_bounds(activated[picked], batch[picked], w_gate_up)
    assert_projection_within_bounds(output[picked], activated[picked], w_down)

    _, normalized, stage_rows = o.mailbox_step(pool, slots, w_gate_up, w_down, norm_weight=norm_weight)
    fp32_rows = o.dense_fp32(normalized, w_gate_up, w_down)
    assert_ffn_parity(output, stage_rows, fp32_rows)
    pure = o.compare(fp32_rows, output.float())
    stage = o.compare(stage_rows, output)
    print(f"max-abs vs fp32 {pure.max_abs:.4e} rel-L2 vs fp32 {pure.rel_l2:.3e} "
          f"max-abs vs stage oracle {stage.max_abs:.4e}", flush=True)
