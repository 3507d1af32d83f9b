"""GPU parity of the MFMA projections (split, stream and tile kernels, K-split tiles).

Bar (tests/parity.py): every projection lies in the bf16 interval that fp32
accumulation of the exact fp64 sum can round to, every activation lies between
the gated-SiLU values of the gate/up roundings reachable that way (+-1 bf16 ulp
for the fp32 exp and divide), and >= 99 % of elements are bit-identical to the
oracle with the reference's rounding points.
"""

from __future__ import annotations

import pytest
import torch

from crosspool_amd import _native, dense
from oracle import ffn_oracle as o
from parity import (
    assert_activated_within_bounds,
    assert_bitwise_equal,
    assert_projection_within_bounds,
    slots_tensor,
    to_device,
)

pytestmark = pytest.mark.gpu

SMALL_SHAPES = [(1024, 3072), (2048, 512), (128, 64)]
ROWS = [1, 3, 16, 17, 32, 33, 64, 65, 128, 200, 256, 300]


def _layer(hidden, intermediate, seed=18):
    w_gate_up, w_down, _ = o.generate_layer(hidden, intermediate, seed)
    return w_gate_up, w_down


@pytest.mark.parametrize("hidden,intermediate", SMALL_SHAPES)
@pytest.mark.parametrize("rows", ROWS)
def test_gate_up_silu_matches_stage_oracle(device, hidden, intermediate, rows):
    x = o.generate_hidden_states(rows, hidden, 17)
    w_gate_up, _ = _layer(hidden, intermediate)
    out = dense.gate_up_silu(to_device(x, device), to_device(w_gate_up, device))
    torch.cuda.synchronize()
    assert_activated_within_bounds(out, x, w_gate_up)


@pytest.mark.parametrize("hidden,intermediate", SMALL_SHAPES)
@pytest.mark.parametrize("rows", ROWS)
def test_down_matches_oracle(device, hidden, intermediate, rows):
    h = o.generate_hidden_states(rows, intermediate, 29)
    _, w_down = _layer(hidden, intermediate)
    out = dense.down(to_device(h, device), to_device(w_down, device))
    torch.cuda.synchronize()
    assert_projection_within_bounds(out, h, w_down)


@pytest.mark.parametrize("rows", [1, 4, 32, 64, 128, 256, 512])
def test_qwen3_8b_projections(device, rows):
    hidden, intermediate = 4096, 12288
    x = o.generate_hidden_states(rows, hidden, 17)
    w_gate_up, w_down = _layer(hidden, intermediate)
    x_d, gu_d, dn_d = to_device(x, device), to_device(w_gate_up, device), to_device(w_down, device)
    activated = dense.gate_up_silu(x_d, gu_d)
    out = dense.down(activated, dn_d)
    torch.cuda.synchronize()
    assert_activated_within_bounds(activated, x, w_gate_up)
    assert_projection_within_bounds(out, activated.cpu(), w_down)


@pytest.mark.parametrize("weight_std", [0.1, 3.0])
def test_reference_linear_case_with_alpha_limit_and_offset(device, weight_std):
    # tests/suites/integration/runtime/ffnagent/test_linear.py:15-21,35-56 (gated, bf16, rows 256,
    # hidden 2048, width 512, inputs randn/sqrt(hidden), weights N(0, 0.1)) with
    # SiluActivation(alpha=1.3) and GateTransform(limit=4, up_offset=-0.5).  The std-3 case
    # drives projections past the limit so both clips are exercised.
    from crosspool_amd.ffn import GateTransform, SiluActivation

    rows, hidden, width = 256, 2048, 512
    generator = torch.Generator().manual_seed(101)
    x = (torch.randn((rows, hidden), generator=generator) / hidden**0.5).to(torch.bfloat16)
    w = (torch.randn((2 * width, hidden), generator=generator) * weight_std).to(torch.bfloat16)
    out = dense.gate_up_silu(
        to_device(x, device),
        to_device(w, device),
        activation=SiluActivation(alpha=1.3),
        gate=GateTransform(limit=4.0, up_offset=-0.5),
    )
    torch.cuda.synchronize()
    assert_activated_within_bounds(out, x, w, alpha=1.3, limit=4.0, up_offset=-0.5)


@pytest.mark.parametrize("rows", [7, 64, 300])
def test_scattering_down_projection_writes_only_its_slots(device, rows):
    hidden, intermediate, pool_rows = 1024, 3072, 512
    h = o.generate_hidden_states(rows, intermediate, 29)
    _, w_down = _layer(hidden, intermediate)
    pool = o.generate_hidden_states(pool_rows, hidden, 31)
    slots = o.generate_slots(pool_rows, rows, 19)
    pool_d = to_device(pool, device)
    dense.down(to_device(h, device), to_device(w_down, device), out=pool_d, slots=slots_tensor(slots, device))
    direct = dense.down(to_device(h, device), to_device(w_down, device))
    torch.cuda.synchronize()
    assert_bitwise_equal(pool_d.cpu(), o.scatter(pool, slots, direct.cpu()))


@pytest.mark.parametrize("rows", [65, 200, 256, 300])
def test_k_split_tiles_with_ragged_ranges(device, rows):
    # K = 3000 (down) splits into ranges of 384 (or 192) columns with a 312- (120-) column
    # last range ending in a partial slab; 200 and 300 rows leave the last row tile partly
    # filled.
    hidden, intermediate = 1024, 3000
    assert "_k" in _native.gemm_variant(rows, hidden, intermediate, False)
    x = o.generate_hidden_states(rows, hidden, 17)
    w_gate_up, w_down = _layer(hidden, intermediate)
    x_d, gu_d, dn_d = to_device(x, device), to_device(w_gate_up, device), to_device(w_down, device)
    activated = dense.gate_up_silu(x_d, gu_d)
    out = dense.down(activated, dn_d)
    again = dense.down(activated, dn_d)
    torch.cuda.synchronize()
    assert_activated_within_bounds(activated, x, w_gate_up)
    assert_projection_within_bounds(out, activated.cpu(), w_down)
    assert_bitwise_equal(out, again)


def test_projections_are_deterministic(device):
    x = to_device(o.generate_hidden_states(256, 4096, 17), device)
    w_gate_up, w_down = (to_device(t, device) for t in _layer(4096, 1024))
    first = dense.down(dense.gate_up_silu(x, w_gate_up), w_down)
    second = dense.down(dense.gate_up_silu(x, w_gate_up), w_down)
    torch.cuda.synchronize()
    assert_bitwise_equal(first, second)


def test_zero_weights_give_zero_output(device):
    # Control Capture Probes are zero weights (src/xpool/runtime/ffnagent/weights.py:265-286).
    x = to_device(o.generate_hidden_states(100, 1024, 17), device)
    zeros_gu = torch.zeros((2 * 512, 1024), dtype=torch.bfloat16, device=device)
    zeros_d = torch.zeros((1024, 512), dtype=torch.bfloat16, device=device)
    out = dense.down(dense.gate_up_silu(x, zeros_gu), zeros_d)
    torch.cuda.synchronize()
    assert torch.equal(out.float().cpu(), torch.zeros((100, 1024)))


def test_variant_selection_covers_every_family(device):
    assert _native.gemm_variant(1, 24576, 4096, True).startswith("split")
    assert _native.gemm_variant(16, 6400, 5120, True).startswith("stream")
    assert _native.gemm_variant(16, 24576, 4096, True).startswith("resident")
    assert _native.gemm_variant(2048, 24576, 4096, True).startswith("tile")
    # the Qwen3-8B cases of test_qwen3_8b_projections reach every tile shape and K splits
    chosen = {_native.gemm_variant(rows, n, k, gated) for rows in (32, 64, 128, 256, 512)
              for n, k, gated in ((24576, 4096, True), (4096, 12288, False))}
    assert {"tile_gated_64x64", "tile_gated_64x128", "tile_gated_128x128", "tile_gated_256x128", "tile_gated_256x256",
            "tile_64x128_k8", "tile_128x128_k8", "tile_256x128_k4"} <= chosen
    # A gated grid of half-full 64-row token tiles under the CU count takes the 64 x 64 tile
    # (Qwen3-8B at 32 rows, not at 64); Qwen3-0.6B at 17 rows keeps the 64 x 128 tile with
    # its K split.
    assert _native.gemm_variant(32, 24576, 4096, True) == "tile_gated_64x64"
    assert _native.gemm_variant(64, 24576, 4096, True) == "tile_gated_64x128"
    assert _native.gemm_variant(17, 6144, 1024, True) == "tile_gated_64x128_k4"
    # The headline sizes of tests/test_gpu_headline.py (config 3 at 1024 / 2048 / 4096 rows,
    # config 5 at 512 / 8192) reach the unsplit tiles, the K-split 256 x 256 down tile and
    # the column splits (a second launch for the trailing columns).
    headline = {_native.gemm_variant(rows, n, k, gated) for (hidden, intermediate), sizes in
                (((4096, 12288), (1024, 2048, 4096)), ((5120, 3200), (512, 8192))) for rows in sizes
                for n, k, gated in ((2 * intermediate, hidden, True), (hidden, intermediate, False))}
    assert {"tile_256x128", "tile_128x128", "tile_256x256", "tile_256x256_k4", "tile_gated_128x128",
            "tile_gated_256x256", "tile_gated_256x256+256x128_n8192", "tile_gated_256x256+64x128_n256",
            "tile_256x256+256x128_n1024"} <= headline


# Ragged geometries of the decode kernels: K not a multiple of their 512-column load
# groups (a partial last K range) or of the tiles' 64-column slabs, N not a multiple of 16
# (weight rows past N), one to many K ranges.  Up to 16 rows a cost model picks the split
# (one token group up to 8 rows, two up to 16) or the stream kernel, from 17 the
# deep-staged small tiles; both decode kernels, and the split kernel with one and with two
# token groups for both projections, must occur on these shapes.
DECODE_SHAPES = [(1032, 1000), (2056, 9992), (4096, 12288), (264, 40), (1544, 2056)]
DECODE_ROWS = [1, 3, 4, 5, 8, 9, 16, 17, 32, 33, 64]


def test_decode_shapes_reach_both_decode_kernels(device):
    names = {_native.gemm_variant(rows, n, k, gated) for hidden, intermediate in DECODE_SHAPES
             for rows in DECODE_ROWS if rows <= 16
             for n, k, gated in ((2 * intermediate, hidden, True), (hidden, intermediate, False))}
    assert {name.split("_")[0] for name in names} == {"split", "stream", "resident"}
    # the split kernel with one and with two token groups, gated and not
    families = {name.rsplit("_k", 1)[0] for name in names if name.startswith("split")}
    assert {"split_t8", "split_t16", "split_gated_t8", "split_gated_t16"} <= families


@pytest.mark.parametrize("hidden,intermediate", DECODE_SHAPES)
@pytest.mark.parametrize("rows", DECODE_ROWS)
def test_decode_projections_on_ragged_geometry(device, hidden, intermediate, rows):
    x = o.generate_hidden_states(rows, hidden, 17)
    w_gate_up, w_down = _layer(hidden, intermediate)
    gu_d, dn_d = to_device(w_gate_up, device), to_device(w_down, device)
    family = ("split", "stream", "resident") if rows <= 16 else ("tile", "resident")
    assert _native.gemm_variant(rows, 2 * intermediate, hidden, True).startswith(family)
    assert _native.gemm_variant(rows, hidden, intermediate, False).startswith(family)
    activated = dense.gate_up_silu(to_device(x, device), gu_d)
    out = dense.down(activated, dn_d)
    # A second call gives the identical bits (fixed-order K reduction).
    again = dense.down(dense.gate_up_silu(to_device(x, device), gu_d), dn_d)
    torch.cuda.synchronize()
    assert_activated_within_bounds(activated, x, w_gate_up)
    assert_projection_within_bounds(out, activated.cpu(), w_down)
    assert_bitwise_equal(again.cpu(), out.cpu())


@pytest.mark.parametrize("rows", [9, 16])
@pytest.mark.parametrize(
    "hidden,intermediate,projection,variant",
    [
        (4096, 12288, "gate_up", "resident_gated_t16_c4"),
        # K = 6000: two parts over the grid (fp32 partials, the ordered reduction with the gated
        # epilogue), the last 128-wide chunk partial and padded chunks past it.
        (6000, 6144, "gate_up", "resident_gated_t16_c3_p2"),
        (5120, 3200, "down", "resident_t16_c4"),  # the Qwen3-32B TP shard's down, one part
    ],
)
def test_resident_projections(device, rows, hidden, intermediate, projection, variant):
    # The token rows held in registers of a one-per-CU grid walking 16-row weight blocks.
    x_rows = o.generate_hidden_states(rows, hidden if projection == "gate_up" else intermediate, 51)
    w_gate_up, w_down = _layer(hidden, intermediate, 52)
    x = to_device(x_rows, device)
    if projection == "gate_up":
        assert _native.gemm_variant(rows, 2 * intermediate, hidden, True) == variant
        w = to_device(w_gate_up, device)
        out = dense.gate_up_silu(x, w)
        again = dense.gate_up_silu(x, w)
        torch.cuda.synchronize()
        assert_activated_within_bounds(out, x_rows, w_gate_up)
    else:
        assert _native.gemm_variant(rows, hidden, intermediate, False) == variant
        w = to_device(w_down, device)
        out = dense.down(x, w)
        again = dense.down(x, w)
        torch.cuda.synchronize()
        assert_projection_within_bounds(out, x_rows, w_down)
    assert_bitwise_equal(again.cpu(), out.cpu())


@pytest.mark.parametrize(
    "n,k,gate_up_variant,down_variant",
    [
        (2304, 512, "tile_gated_256x256+64x128_n256", "tile_256x256+64x128_n256"),
        # The second launch's 128 columns are half a 256-wide weight tile of the first shape.
        (2176, 320, "tile_gated_256x256+64x128_n128", "tile_256x256+64x128_n128"),
    ],
)
def test_column_split_projections(device, n, k, gate_up_variant, down_variant):
    # 8192 rows: 32 token tiles, so the first 2048 weight rows on 256 x 256 tiles are exactly
    # one round of 256 workgroups and the remaining columns go to a second launch on smaller
    # tiles (its weights, and its output columns: half as many for gate_up).
    rows = 8192
    print(f"column split n={n} k={k}", flush=True)
    assert _native.gemm_variant(rows, n, k, True) == gate_up_variant
    assert _native.gemm_variant(rows, n, k, False) == down_variant
    assert _native.gemm_workspace_bytes(rows, n, k, True) == 0 and _native.gemm_workspace_bytes(rows, n, k, False) == 0
    x_rows = o.generate_hidden_states(rows, k, 71)
    w_gate_up, _ = _layer(k, n // 2, 72)
    _, w_down = _layer(n, k, 73)
    x = to_device(x_rows, device)
    activated = dense.gate_up_silu(x, to_device(w_gate_up, device))
    out = dense.down(x, to_device(w_down, device))
    torch.cuda.synchronize()
    assert_activated_within_bounds(activated, x_rows, w_gate_up)
    assert_projection_within_bounds(out, x_rows, w_down)


@pytest.mark.parametrize("rows", [1, 16, 128])
def test_projection_rounds_to_nearest_even(device, rows):
    # Every output is a + b * c with a, b, c chosen so the fp32 sum is exact and often lands
    # exactly halfway between two bf16 values: the stored bits must be the round-to-nearest-
    # even of that sum (what torch's float -> bf16 conversion produces), for the split, stream
    # and tile kernels alike.
    hidden, intermediate = 64, 64
    generator = torch.Generator().manual_seed(7)
    mantissa = torch.randint(0, 128, (rows,), generator=generator).double()
    a = (1.0 + mantissa / 128) * torch.where(torch.rand(rows, generator=generator) < 0.5, -1.0, 1.0)
    b = torch.tensor([2.0**-9, -(2.0**-9), 3 * 2.0**-10, 2.0**-10, 2.0**-20, 0.0, 5 * 2.0**-10, -(2.0**-8)])
    b = b[torch.arange(rows) % len(b)]
    h = torch.zeros((rows, intermediate), dtype=torch.float64)
    h[:, 0], h[:, 1] = a, b
    c = torch.tensor([2.0 ** (-(n % 4)) * (-1 if n % 3 == 0 else 1) for n in range(hidden)], dtype=torch.float64)
    w = torch.zeros((hidden, intermediate), dtype=torch.float64)
    w[:, 0], w[:, 1] = 1.0, c
    h_bf, w_bf = h.to(torch.bfloat16), w.to(torch.bfloat16)
    assert torch.equal(h_bf.double(), h) and torch.equal(w_bf.double(), w)
    expected = (h @ w.t()).float().to(torch.bfloat16)  # exact in fp32, one rounding
    out = dense.down(to_device(h_bf, device), to_device(w_bf, device))
    torch.cuda.synchronize()
    assert_bitwise_equal(out.cpu(), expected)
