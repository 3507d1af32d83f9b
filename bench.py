"""FFN-layer throughput of the MI355X FfnAgent path at the Qwen3-8B shape.

One step = one replay of the Dense mailbox step's GraphTemplate (its captured
kernels launched on the Lane stream) for a batch of T tokens: gather T seeded slots of an 8192-slot bf16 mailbox with the fused
RMSNorm, gate_up [4096 -> 2 x 12288] + SiLU*mul, down [12288 -> 4096],
scatter back into the same slots.  Inputs are resident in HBM before timing.

Prints ONE JSON line: the headline at T = --tokens (default 2048, the
MFMA-bound north-star point), a ``decode`` entry at T = 32 (HBM-bound: the layer,
and the kernel-level gate_up's roofline beside the name of the kernel the layer runs), the
batch sweep of BASELINE config 3, the roofline of the dominant kernel
(measured with HIP events on the Lane stream it runs on) and the CPU
baseline (the oracle's torch-CPU restatement on the host cores); beside them the
other configs, a Qwen3-30B-A3B-shaped MoE layer with bf16 (``moe``) and fp16
(``moe_fp16``) payloads, and the Qwen3-8B layer with fp16 payloads (``dense_fp16``).

``--kernels-only`` instead launches just the kernels whose hardware counters
the roofline's ``traffic`` figure comes from (a byte copy of known size for
calibration, then gate_up at the headline and decode sizes), and layer replays
at 16 rows and one row, for ``rocprofv3 --pmc`` runs; ``profiles/traffic.json``
records their result.

``--ceilings`` instead measures the hardware limits the kernels are judged
against (libxpool_probes.so): a pure-MFMA loop, two HBM read patterns, the
GPU idle time a hipGraphLaunch adds per replay, the cost of a grid-wide
dependency (a kernel boundary against an in-kernel counter handoff), and
torch.matmul (hipBLASLt) on the headline's two product shapes, and prints them
as one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO_ROOT))

HIDDEN, INTERMEDIATE = 4096, 12288
POOL_SLOTS = 8192
SWEEP = (1, 4, 16, 32, 64, 256, 1024, 2048, 4096)
GRAPH_DISPATCH_TOKENS = (1, 32, 2048)  # replays timed through the instantiated hipGraph too
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
# Copies of the gate_up weights the decode roofline rotates through (3 x 201 MB exceeds
# the 256 MB last-level cache, so every launch streams its weights from HBM).
DECODE_WEIGHT_SETS = 3
CALIBRATION_COPY_BYTES = 256 << 20
# TP partial fold measured at BASELINE config 5 (Qwen3-32B, 8 shards of H = 5120, T = 8192).
TP_REDUCE_PARTIALS = 8
TP_REDUCE_SHAPE = (8192, 5120)
TP_REDUCE_LAUNCHES = 20
TRAFFIC_FILE = REPO_ROOT / "profiles" / "traffic.json"
# Qwen3-0.6B FFN (hidden, intermediate) x 28 layers, and its batch sizes.
STACK_SHAPE = (1024, 3072, 28)
STACK_TOKENS = (1, 8, 32, 128, 256)
# one of 8 tensor-parallel shards of a Qwen3-32B FFN, its batch sizes, and
# the weight copies rotated at HBM-bound sizes (4 x 98 MB exceeds the last-level cache).
SHARD_SHAPE = (5120, 3200)
SHARD_TOKENS = (8, 512, 8192)
SHARD_COPIES = 4
# two co-located models on two Lanes, ragged 1..512 rows per step each.
COLOCATED_SHAPES = ((2048, 6144), (2560, 9728))
COLOCATED_MAX_ROWS = 512
COLOCATED_LAYERS = 3  # distinct weight sets per model, rotated per step
COLOCATED_STEPS = 60
# Qwen3-30B-A3B MoE layer (hidden, moe_intermediate, experts, top-k) and its token points.
MOE_SHAPE = (2048, 768, 128, 8)
MOE_TOKENS = (1, 32, 2048)


def parse_args() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--tokens", type=int, default=2048)
    parser.add_argument("--decode-tokens", type=int, default=32)
    parser.add_argument("--sweep-steps", type=int, default=30)
    parser.add_argument("--no-sweep", action="store_true")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--kernels-only", action="store_true", help="launch only the profiled kernels, then exit")
    parser.add_argument("--ceilings", action="store_true", help="measure the hardware ceilings, then exit")
    parser.add_argument("--prewarm-seconds", type=float, default=2.0,
                        help="untimed replays before the headline's warmup, so clocks are at steady state")
    return parser.parse_args()


def measured_traffic(variant: str, tokens: int) -> float | None:
    """HBM bytes per launch of `variant` at `tokens` from the committed counter summary."""

    try:
        entries = json.loads(TRAFFIC_FILE.read_text())["kernels"]
    except (OSError, ValueError, KeyError):
        return None
    for entry in entries:
        if entry.get("kernel") == variant and entry.get("tokens") == tokens:
            return float(entry["bytes_per_launch"])
    return None


def layer_flops(tokens: int) -> float:
    return 6.0 * tokens * HIDDEN * INTERMEDIATE


def layer_bytes(tokens: int) -> float:
    # weights + norm weight + gathered rows + scattered rows + int32 slot ids
    return 6.0 * HIDDEN * INTERMEDIATE + 2 * HIDDEN + 4.0 * tokens * HIDDEN + 4.0 * tokens


def gate_up_flops(tokens: int) -> float:
    return 4.0 * tokens * HIDDEN * INTERMEDIATE


def gate_up_bytes(tokens: int) -> float:
    # i_proj weights + the gathered batch read + the activated intermediate written
    return 4.0 * HIDDEN * INTERMEDIATE + 2.0 * tokens * HIDDEN + 2.0 * tokens * INTERMEDIATE


def mfma_ceiling(stream) -> dict:
    """The bf16 matrix rate a pure-MFMA loop sustains on random operands (no memory
    traffic), measured on `stream` with HIP events, and the shader clock the chip held."""

    import ctypes

    import torch

    from crosspool_amd import build

    probes = ctypes.CDLL(str(build.PROBE_LIBRARY))
    clocks = torch.zeros(2, dtype=torch.int64, device=stream.device)
    workgroups, rounds = 2048, 4000

    def launch() -> None:
        status = probes.xp_probe_mfma(workgroups, rounds, 1, ctypes.c_void_p(clocks.data_ptr()),
                                      ctypes.c_void_p(stream.cuda_stream))
        if status != 0:
            raise RuntimeError(f"MFMA probe launch failed with status {status}")

    launch()
    begin = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    begin.record(stream)
    launch()
    end.record(stream)
    end.synchronize()
    seconds = begin.elapsed_time(end) / 1e3
    cycles, ticks = (int(value) for value in clocks.cpu())
    tflops = workgroups * 4 * rounds * 8 * 2.0 * 32 * 32 * 16 / seconds / 1e12
    return {"tflops": round(tflops, 1), "frac_of_peak": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "clock_ghz": round(cycles / (ticks * 10.0), 3) if ticks > 0 else None}


def run_ceilings(device) -> dict:
    """Hardware limits measured with HIP events on the current stream (see the module doc)."""

    import ctypes

    import torch

    from crosspool_amd import build
    from crosspool_amd.agent import FfnAgent
    from crosspool_amd.weights import DenseFfnWeights

    probes = ctypes.CDLL(str(build.PROBE_LIBRARY))
    stream = torch.cuda.current_stream(device)
    handle = ctypes.c_void_p(stream.cuda_stream)

    def per_launch(launch, repeats: int) -> float:
        for _ in range(2):
            launch()
        begin = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        begin.record(stream)
        for index in range(repeats):
            launch(index)
        end.record(stream)
        end.synchronize()
        return begin.elapsed_time(end) / 1e3 / repeats

    def checked(status: int) -> None:
        if status != 0:
            raise RuntimeError(f"probe launch failed with status {status}")

    result: dict = {}
    # bf16 MFMA: 4-wave workgroups, 8 independent 32x32x16 chains per wave, with low-entropy
    # constant operands and with rotating random operands (the switching power of a GEMM's
    # main loop); the clock comes from workgroup 0's shader-cycle and 100 MHz counters.
    clocks = torch.zeros(2, dtype=torch.int64, device=device)
    mfma = []
    for random in (0, 1):
        for workgroups, rounds in ((1024, 20000), (2048, 20000)):
            seconds = per_launch(lambda index=0: checked(probes.xp_probe_mfma(
                workgroups, rounds, random, ctypes.c_void_p(clocks.data_ptr()), handle)), 5)
            cycles, ticks = (int(value) for value in clocks.cpu())
            flops = workgroups * 4 * rounds * 8 * 2.0 * 32 * 32 * 16
            mfma.append({"operands": "random" if random else "constant", "workgroups": workgroups,
                         "tflops": round(flops / seconds / 1e12, 1),
                         "clock_ghz": round(cycles / (ticks * 10.0), 3) if ticks > 0 else None})
    best = max(point["tflops"] for point in mfma)
    best_random = max(point["tflops"] for point in mfma if point["operands"] == "random")
    result["mfma_bf16"] = {"points": mfma, "best_tflops": best, "frac_of_2500": round(best / MFMA_BF16_PEAK_TFLOPS, 4),
                           "best_random_tflops": best_random,
                           "random_frac_of_2500": round(best_random / MFMA_BF16_PEAK_TFLOPS, 4)}

    # HBM reads: a 4 GiB buffer (far past the 256 MB last-level cache), 1 KB per wave
    # instruction, plain loads and loads with the nontemporal hint.
    buffer = torch.empty(4 << 30, dtype=torch.uint8, device=device)
    contiguous = []
    for nontemporal in (0, 1):
        for workgroups in (2048, 8192, 32768):
            seconds = per_launch(lambda index=0: checked(probes.xp_probe_read_contiguous(
                ctypes.c_void_p(buffer.data_ptr()), ctypes.c_uint64(buffer.numel()), workgroups, nontemporal,
                handle)), 10)
            contiguous.append({"workgroups": workgroups, "nontemporal": bool(nontemporal),
                               "gbs": round(buffer.numel() / seconds / 1e9, 1)})
    del buffer
    # The decode weight-stream pattern over three copies of the Qwen3-8B gate_up matrix
    # ([24576, 4096] bf16, 201 MB each, rotated so each launch streams from HBM).
    rows, row_bytes = 2 * INTERMEDIATE, 2 * HIDDEN
    copies = [torch.empty(rows * row_bytes, dtype=torch.uint8, device=device) for _ in range(3)]
    row_points = []
    for pattern, name in ((0, "half_lines"), (3, "half_lines_nt"), (1, "lines"), (2, "lines_nt")):
        for ranges in (1, 2, 4, 8):
            seconds = per_launch(lambda index=0: checked(probes.xp_probe_read_rows(
                ctypes.c_void_p(copies[index % 3].data_ptr()), ctypes.c_int64(rows), ctypes.c_int64(row_bytes),
                ranges, pattern, handle)), 30)
            row_points.append({"pattern": name, "ranges": ranges, "workgroups": (rows // 16 + 7) // 8 * ranges,
                               "gbs": round(rows * row_bytes / seconds / 1e9, 1)})
    del copies
    best_read = max(point["gbs"] for point in contiguous + row_points)
    result["hbm_read"] = {"contiguous_4gib": contiguous, "weight_rows_qwen3_8b_gate_up": row_points,
                          "best_gbs": best_read, "frac_of_8000": round(best_read / HBM_PEAK_GBS, 4)}

    # GPU time a hipGraphLaunch adds per replay: one Qwen3-0.6B layer at one row replayed
    # back to back through direct kernel launches and through its instantiated hipGraph.
    generator = torch.Generator(device=device).manual_seed(18)
    graph_points = {}
    for graph_dispatch in (False, True):
        with FfnAgent(device, graph_dispatch=graph_dispatch) as agent:
            agent.register_layer(
                instance_index=0, layer_ordinal=0,
                weights=DenseFfnWeights.from_tensors(
                    (torch.randn((6144, 1024), device=device, generator=generator) * 0.02).bfloat16(),
                    (torch.randn((1024, 3072), device=device, generator=generator) * 0.02).bfloat16()),
            )
            agent.materialize(maximum_row_capacity=1)
            lane = agent.lanes[0]
            pool = torch.randn((64, 1024), device=device, generator=generator).bfloat16()
            slots = torch.arange(1, dtype=torch.int32, device=device)
            lane_stream = lane.stream
            begin = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            for _ in range(20):
                lane.replay(instance_index=0, layer_ordinal=0, pool=pool, slots=slots, stream=lane_stream)
            begin.record(lane_stream)
            for _ in range(200):
                lane.replay(instance_index=0, layer_ordinal=0, pool=pool, slots=slots, stream=lane_stream)
            end.record(lane_stream)
            end.synchronize()
            graph_points["graph" if graph_dispatch else "direct"] = begin.elapsed_time(end) * 1e3 / 200
    result["replay_us_qwen3_0_6b_t1"] = {key: round(value, 2) for key, value in graph_points.items()}
    result["graph_launch_extra_us"] = round(graph_points["graph"] - graph_points["direct"], 2)

    # A grid-wide dependency: empty kernels back to back, and a producer -> consumer handoff
    # across a kernel boundary and inside one launch (one counter, or a counter per 8
    # producers).
    result["empty_kernel_us"] = round(per_launch(
        lambda index=0: checked(probes.xp_probe_empty(256, handle)), 200) * 1e6, 2)
    words = torch.zeros(512 * 8, dtype=torch.int32, device=device)
    counters = torch.zeros(64 * 32, dtype=torch.int32, device=device)
    flag = torch.zeros(1, dtype=torch.int32, device=device)
    handoff = []
    for producers, consumers in ((192, 64), (192, 256), (512, 64), (512, 256)):
        point = {"producers": producers, "consumers": consumers}
        for mode, name in ((0, "two_kernels_us"), (1, "one_launch_one_counter_us"),
                           (2, "one_launch_counter_per_8_us")):
            counters.zero_()
            epoch = [0]

            def launch(index=0, mode=mode, producers=producers, consumers=consumers):
                epoch[0] += 1
                checked(probes.xp_probe_handoff(
                    producers, consumers, mode, ctypes.c_void_p(words.data_ptr()),
                    ctypes.c_void_p(counters.data_ptr()), ctypes.c_uint32(epoch[0]), ctypes.c_uint32(epoch[0]),
                    ctypes.c_void_p(flag.data_ptr()), handle))

            point[name] = round(per_launch(launch, 200) * 1e6, 2)
        handoff.append(point)
    torch.cuda.synchronize(device)
    result["handoff"] = {"points": handoff, "flag": int(flag.item())}

    # The library GEMM on the headline shapes: torch.matmul (hipBLASLt) of bf16 [2048, 4096] x
    # [4096, 24576] (gate_up's product, bf16 output of all 2I columns, no activation) and
    # [2048, 12288] x [12288, 4096] (down's), N(0, 1) activations and N(0, 0.02) weights as
    # in the headline, timed back to back.
    library = []
    for name, m, k, n in (("gate_up_shape", 2048, HIDDEN, 2 * INTERMEDIATE), ("down_shape", 2048, INTERMEDIATE, HIDDEN)):
        a = torch.randn((m, k), device=device, generator=generator).bfloat16()
        b = (torch.randn((n, k), device=device, generator=generator) * 0.02).bfloat16()
        out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
        bt = b.t()
        seconds = per_launch(lambda index=0: torch.matmul(a, bt, out=out), 20)
        library.append({"product": name, "m": m, "k": k, "n": n, "us": round(seconds * 1e6, 1),
                        "tflops": round(2.0 * m * n * k / seconds / 1e12, 1)})
        del a, b, out, bt
    result["hipblaslt_matmul"] = library
    return result


def main() -> int:
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one MI355X: the FfnAgent path here is single-GPU (no collectives); "
            "run it with --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    from crosspool_amd import _native, dense
    from crosspool_amd.agent import FfnAgent
    from crosspool_amd.execution import derive_payload_row_capacities, select_capacity
    from crosspool_amd.weights import DenseFfnWeights
    from oracle import ffn_oracle as o

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.ceilings:
        print(json.dumps({"ceilings": run_ceilings(device)}), flush=True)
        return 0
    max_tokens = max(SWEEP + (args.tokens, args.decode_tokens))

    pool_cpu = o.generate_hidden_states(POOL_SLOTS, HIDDEN, 17)
    w_gate_up, w_down, norm_weight = o.generate_layer(HIDDEN, INTERMEDIATE, 18)
    slots_cpu = o.generate_slots(POOL_SLOTS, max_tokens, 19)
    pool = pool_cpu.to(device)
    slots = torch.from_numpy(slots_cpu).to(device)
    weights = DenseFfnWeights.from_tensors(w_gate_up.to(device), w_down.to(device))
    norm = norm_weight.to(device)

    agent = FfnAgent(device)
    agent.register_layer(instance_index=0, layer_ordinal=0, weights=weights, norm_weight=norm, eps=1e-6)
    # Layer 1: the same values in a second copy.  Layer timings at HBM-bound sizes alternate
    # the two layers, so each replay streams its 302 MB of weights from HBM instead of
    # partly from the 256 MB last-level cache, as a stack of distinct layers does.
    agent.register_layer(
        instance_index=0, layer_ordinal=1,
        weights=DenseFfnWeights.from_tensors(weights.i_proj.values.clone(), weights.o_proj.values.clone()),
        norm_weight=norm, eps=1e-6,
    )
    agent.materialize(maximum_row_capacity=max_tokens)
    lane = agent.lanes[0]
    torch.cuda.synchronize()

    def replay(tokens: int, ordinal: int = 0) -> None:
        lane.replay(instance_index=0, layer_ordinal=ordinal, pool=pool, slots=slots, rows=tokens, stream=lane.stream)

    def time_replays(tokens: int, steps: int, warmup: int, prewarm_seconds: float = 0.0) -> float:
        ordinals = (0, 1) if tokens <= 256 else (0,)
        deadline = time.perf_counter() + prewarm_seconds
        while time.perf_counter() < deadline:  # untimed: clocks reach steady state
            for _ in range(10):
                replay(tokens)
            torch.cuda.synchronize()
        for step in range(warmup):
            replay(tokens, ordinals[step % len(ordinals)])
        torch.cuda.synchronize()
        start = time.perf_counter()
        for step in range(steps):
            replay(tokens, ordinals[step % len(ordinals)])
        torch.cuda.synchronize()
        return (time.perf_counter() - start) / steps

    tokens = args.tokens

    # ---------------------------------------------------------------- dominant kernel (events)
    decode_weight_sets = [weights.i_proj.values] + [
        weights.i_proj.values.clone() for _ in range(DECODE_WEIGHT_SETS - 1)
    ]

    def gate_up_launches(tokens: int, steps: int) -> float:
        """Average seconds per gate_up launch (its reduction launch included when it has
        one), timed with HIP events on the Lane stream.  HBM-bound sizes rotate through
        weight copies larger than the last-level cache together."""

        x = torch.empty((tokens, HIDDEN), dtype=torch.bfloat16, device=device)
        dense.gather_rmsnorm(pool, slots[:tokens], norm_weight=norm, out=x, stream=lane.stream)
        h = torch.empty((tokens, INTERMEDIATE), dtype=torch.bfloat16, device=device)
        sets = [weights.i_proj.values] if tokens > 64 else decode_weight_sets
        for index in range(3):
            dense.gate_up_silu(x, sets[index % len(sets)], out=h, stream=lane.stream)
        begin = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        begin.record(lane.stream)
        for index in range(steps):
            dense.gate_up_silu(x, sets[index % len(sets)], out=h, stream=lane.stream)
        end.record(lane.stream)
        end.synchronize()
        return begin.elapsed_time(end) / 1e3 / steps

    def kernel_roofline(tokens: int, steps: int) -> dict:
        per_launch = gate_up_launches(tokens, steps)
        variant = _native.gemm_variant(tokens, 2 * INTERMEDIATE, HIDDEN, True)
        traffic = measured_traffic(variant, tokens)
        # Up to 64 rows the projection streams its weights (HBM-bound); above, MFMA-bound.
        if tokens > 64:
            achieved = gate_up_flops(tokens) / per_launch / 1e12
            ceiling = mfma_ceiling(lane.stream)
            return {
                "kernel": variant, "tokens": tokens, "bound": "mfma", "achieved": round(achieved, 1),
                "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                "traffic": traffic, "avg_launch_us": round(per_launch * 1e6, 2),
                "algorithmic_flops": gate_up_flops(tokens),
                "sustained_mfma_random_operands": {**ceiling,
                                                   "kernel_frac_of_it": round(achieved / ceiling["tflops"], 4)},
            }
        achieved = gate_up_bytes(tokens) / per_launch / 1e9
        return {
            "kernel": variant, "tokens": tokens, "bound": "hbm", "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic, "avg_launch_us": round(per_launch * 1e6, 2),
            "algorithmic_bytes": gate_up_bytes(tokens),
        }

    if args.kernels_only:
        # Calibration copy of known size, then the roofline kernels, a few launches each.
        source = torch.empty(CALIBRATION_COPY_BYTES, dtype=torch.uint8, device=device)
        target = torch.empty_like(source)
        for _ in range(5):
            dense.copy_bytes(target, source, stream=lane.stream)
        # gate_up at the headline and decode sizes (the roofline's traffic), then whole layer
        # replays at 16 rows and one row, whose gate_up kernels (the resident kernel, the
        # persistent split kernel, both with the gather fused) exist only in a Dense step
        for t in (tokens, args.decode_tokens):
            gate_up_launches(t, 6)
        for t in (16, 1):
            for step in range(6):
                replay(t, step % 2)
        torch.cuda.synchronize()
        agent.close()
        print(json.dumps({"kernels_only": True, "copy_bytes": CALIBRATION_COPY_BYTES,
                          "gate_up_tokens": [tokens, args.decode_tokens], "layer_replay_tokens": [16, 1]}),
              flush=True)
        return 0

    # ---------------------------------------------------------------- headline
    seconds = time_replays(tokens, args.steps, args.warmup, prewarm_seconds=args.prewarm_seconds)
    agent.check_health()
    roofline = kernel_roofline(tokens, max(20, min(args.steps, 200)))

    # ---------------------------------------------------------------- decode point
    decode_seconds = time_replays(args.decode_tokens, args.steps, args.warmup, prewarm_seconds=0.5)
    decode = {
        "tokens": args.decode_tokens,
        "tokens_per_s": round(args.decode_tokens / decode_seconds, 1),
        "us_per_layer": round(decode_seconds * 1e6, 2),
        "layer_hbm_frac": round(layer_bytes(args.decode_tokens) / decode_seconds / 1e9 / HBM_PEAK_GBS, 4),
        # The kernel-level gate_up at this size (no gather); the Dense step may run another
        # kernel for it (the gather fused into the resident kernel at 9-32 rows), named here.
        "roofline": kernel_roofline(args.decode_tokens, 200),
        "layer_gate_up": _native.dense_gate_up_variant(args.decode_tokens, HIDDEN, INTERMEDIATE),
    }

    # ---------------------------------------------------------------- sweep
    sweep = []
    if not args.no_sweep:
        for t in SWEEP:
            s = time_replays(t, args.sweep_steps, 5)
            hbm = layer_bytes(t) / s / 1e9 / HBM_PEAK_GBS
            mfma = layer_flops(t) / s / 1e12 / MFMA_BF16_PEAK_TFLOPS
            sweep.append({
                "tokens": t, "us": round(s * 1e6, 2), "tokens_per_s": round(t / s, 1),
                "hbm_frac": round(hbm, 4), "mfma_frac": round(mfma, 4),
            })
    agent.check_health()

    # ---------------------------------------------------------------- graph dispatch
    # The same replays launched as the template's instantiated hipGraph (the reference's
    # design: one captured graph per layer signature) against the default direct launches.
    graph_dispatch = None
    if not args.no_sweep:
        points = []
        for t in GRAPH_DISPATCH_TOKENS:
            direct_s = time_replays(t, args.sweep_steps, 5)
            lane.set_graph_dispatch(True)
            graph_s = time_replays(t, args.sweep_steps, 5)
            lane.set_graph_dispatch(False)
            points.append({"tokens": t, "direct_us": round(direct_s * 1e6, 2), "graph_us": round(graph_s * 1e6, 2),
                           "graph_extra_us": round((graph_s - direct_s) * 1e6, 2)})
        graph_dispatch = {"execution": "hipGraphLaunch of the template's instantiated graph per replay "
                                       "(changed kernel nodes rebound) against direct kernel launches",
                          "points": points}
    agent.check_health()

    # ---------------------------------------------------------------- TP partial fold
    # xp_reduce_partials at the Qwen3-32B 1/8-shard partial shape (
    # T = 8192): 8 bf16 partials folded in rank order; (8 + 1) x 2 bytes per element.
    tp_reduce = None
    if not args.no_sweep:
        from crosspool_amd.delivery import reduce_tp_partials

        partials = [torch.randn(TP_REDUCE_SHAPE, device=device).bfloat16() for _ in range(TP_REDUCE_PARTIALS)]
        folded = torch.empty_like(partials[0])
        for _ in range(3):
            reduce_tp_partials(partials, out=folded, stream=lane.stream)
        begin = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        begin.record(lane.stream)
        for _ in range(TP_REDUCE_LAUNCHES):
            reduce_tp_partials(partials, out=folded, stream=lane.stream)
        end.record(lane.stream)
        end.synchronize()
        per_launch = begin.elapsed_time(end) / 1e3 / TP_REDUCE_LAUNCHES
        moved = (TP_REDUCE_PARTIALS + 1) * folded.numel() * 2
        tp_reduce = {
            "partials": TP_REDUCE_PARTIALS, "shape": list(TP_REDUCE_SHAPE), "us": round(per_launch * 1e6, 2),
            "achieved": round(moved / per_launch / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(moved / per_launch / 1e9 / HBM_PEAK_GBS, 4), "algorithmic_bytes": moved,
        }
        del partials, folded

    # ---------------------------------------------------------------- config 2 stack
    # the 28-layer Qwen3-0.6B FFN stack, independent weights per layer,
    # T rows of a 4096-slot mailbox; one step = all 28 layers replayed in order on the Lane,
    # timed as one captured hipGraph per step (and, for reference, issued from the host).
    stack = None
    if not args.no_sweep:
        s_hidden, s_inter, s_layers = STACK_SHAPE
        generator = torch.Generator(device=device).manual_seed(18)
        stack_agent = FfnAgent(device)
        for ordinal in range(s_layers):
            stack_agent.register_layer(
                instance_index=0, layer_ordinal=ordinal,
                weights=DenseFfnWeights.from_tensors(
                    (torch.randn((2 * s_inter, s_hidden), device=device, generator=generator) * 0.02).bfloat16(),
                    (torch.randn((s_hidden, s_inter), device=device, generator=generator) * 0.02).bfloat16(),
                ),
                norm_weight=(1 + 0.1 * torch.randn(s_hidden, device=device, generator=generator)).bfloat16(),
            )
        stack_agent.materialize(maximum_row_capacity=max(STACK_TOKENS))
        stack_lane = stack_agent.lanes[0]
        stack_pool = torch.randn((4096, s_hidden), device=device, generator=generator).bfloat16()
        stack_slots = torch.randperm(4096, device=device, generator=generator)[: max(STACK_TOKENS)].int()
        stack = {"layers": s_layers, "hidden": s_hidden, "intermediate": s_inter, "points": []}
        for t in STACK_TOKENS:
            def stack_step() -> None:
                for ordinal in range(s_layers):
                    stack_lane.replay(instance_index=0, layer_ordinal=ordinal, pool=stack_pool, slots=stack_slots,
                                      rows=t, stream=stack_lane.stream)

            for _ in range(3):
                stack_step()
            torch.cuda.synchronize()
            started = time.perf_counter()
            for _ in range(args.sweep_steps):
                stack_step()
            torch.cuda.synchronize()
            eager_seconds = (time.perf_counter() - started) / args.sweep_steps
            # The same 28 replays captured into one hipGraph, as a serving step under graph
            # capture issues them: one launch per stack step instead of ~100 from the host.
            graph = torch.cuda.CUDAGraph()
            capture = torch.cuda.Stream()
            capture.wait_stream(torch.cuda.current_stream())
            with torch.cuda.graph(graph, stream=capture):
                for ordinal in range(s_layers):
                    stack_lane.replay(instance_index=0, layer_ordinal=ordinal, pool=stack_pool, slots=stack_slots,
                                      rows=t, stream=torch.cuda.current_stream())
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            started = time.perf_counter()
            for _ in range(args.sweep_steps):
                graph.replay()
            torch.cuda.synchronize()
            step_seconds = (time.perf_counter() - started) / args.sweep_steps
            del graph
            stack_bytes = s_layers * (6.0 * s_hidden * s_inter + 2 * s_hidden + 4.0 * t * s_hidden + 4.0 * t)
            stack["points"].append({
                "tokens": t, "us_per_stack": round(step_seconds * 1e6, 2),
                "us_per_layer": round(step_seconds * 1e6 / s_layers, 2),
                "tokens_per_s": round(t / step_seconds, 1),
                "hbm_frac": round(stack_bytes / step_seconds / 1e9 / HBM_PEAK_GBS, 4),
                "host_issued_us_per_stack": round(eager_seconds * 1e6, 2),
            })
        stack_agent.check_health()
        stack_agent.close()
        del stack_pool

    # ---------------------------------------------------------------- config 5 shard
    # the unreduced partial of one Qwen3-32B TP shard (hidden 5120, shard
    # intermediate 3200) at T = 8, 512, 8192 rows of an 8192-slot mailbox, written to a
    # separate output mailbox; weight copies rotated per replay.
    shard = None
    if not args.no_sweep:
        p_hidden, p_inter = SHARD_SHAPE
        generator = torch.Generator(device=device).manual_seed(18)
        shard_agent = FfnAgent(device)
        base_gate_up = (torch.randn((2 * p_inter, p_hidden), device=device, generator=generator) * 0.02).bfloat16()
        base_down = (torch.randn((p_hidden, p_inter), device=device, generator=generator) * 0.02).bfloat16()
        for ordinal in range(SHARD_COPIES):
            shard_agent.register_layer(
                instance_index=0, layer_ordinal=ordinal,
                weights=DenseFfnWeights.from_tensors(base_gate_up.clone(), base_down.clone()),
            )
        shard_agent.materialize(maximum_row_capacity=max(SHARD_TOKENS))
        shard_lane = shard_agent.lanes[0]
        shard_pool = torch.randn((max(SHARD_TOKENS), p_hidden), device=device, generator=generator).bfloat16()
        shard_out = torch.empty_like(shard_pool)
        shard_slots = torch.randperm(max(SHARD_TOKENS), device=device, generator=generator).int()
        shard = {"hidden": p_hidden, "shard_intermediate": p_inter, "tp_shards": 8, "points": []}
        for t in SHARD_TOKENS:
            def shard_replay(step: int) -> None:
                shard_lane.replay(instance_index=0, layer_ordinal=step % SHARD_COPIES, pool=shard_pool,
                                  out_pool=shard_out, slots=shard_slots, rows=t, stream=shard_lane.stream)

            steps = max(20, min(200, 400000 // t))
            for step in range(10):
                shard_replay(step)
            torch.cuda.synchronize()
            started = time.perf_counter()
            for step in range(steps):
                shard_replay(step)
            torch.cuda.synchronize()
            per = (time.perf_counter() - started) / steps
            p_bytes = 6.0 * p_hidden * p_inter + 4.0 * t * p_hidden + 4.0 * t
            p_flops = 6.0 * t * p_hidden * p_inter
            shard["points"].append({
                "tokens": t, "us": round(per * 1e6, 2), "tokens_per_s": round(t / per, 1),
                "hbm_frac": round(p_bytes / per / 1e9 / HBM_PEAK_GBS, 4),
                "mfma_frac": round(p_flops / per / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                "bound": "hbm" if t <= 64 else "mfma",
            })
        shard_agent.check_health()
        shard_agent.close()
        del shard_pool, shard_out, base_gate_up, base_down

    # ---------------------------------------------------------------- config 4 co-location
    # a Qwen3-1.7B-shaped and a Qwen3-4B-shaped layer on one GPU, each on
    # its own Lane (own stream).  Per step each instance submits T ~ U{1..512} rows (seeded)
    # from a disjoint half of an 8192-slot mailbox of its width; both Lanes replay
    # concurrently.  Each model rotates through distinct weight copies.  Reported: per-model
    # tokens/s with the Lanes concurrent and alone, and the combined HBM fraction.
    colocated = None
    if not args.no_sweep:
        import numpy as np

        rng = np.random.default_rng(7)
        generator = torch.Generator(device=device).manual_seed(18)
        co_agent = FfnAgent(device, executor_lane_count=2)
        co_pools, co_slots = [], []
        for instance, (c_hidden, c_inter) in enumerate(COLOCATED_SHAPES):
            for ordinal in range(COLOCATED_LAYERS):
                co_agent.register_layer(
                    instance_index=instance, layer_ordinal=ordinal,
                    weights=DenseFfnWeights.from_tensors(
                        (torch.randn((2 * c_inter, c_hidden), device=device, generator=generator) * 0.02).bfloat16(),
                        (torch.randn((c_hidden, c_inter), device=device, generator=generator) * 0.02).bfloat16()),
                    norm_weight=(1 + 0.1 * torch.randn(c_hidden, device=device, generator=generator)).bfloat16(),
                )
            co_pools.append(torch.randn((8192, c_hidden), device=device, generator=generator).bfloat16())
            first = instance * 4096
            co_slots.append((first + torch.randperm(4096, device=device, generator=generator)).int())
        co_agent.materialize(maximum_row_capacity=COLOCATED_MAX_ROWS)
        rows_per_step = rng.integers(1, COLOCATED_MAX_ROWS + 1, size=(COLOCATED_STEPS, 2))

        def run_steps(instances: tuple[int, ...]) -> float:
            torch.cuda.synchronize()
            started = time.perf_counter()
            for step in range(COLOCATED_STEPS):
                for instance in instances:
                    lane = co_agent.lanes[instance]
                    lane.replay(instance_index=instance, layer_ordinal=step % COLOCATED_LAYERS,
                                pool=co_pools[instance], slots=co_slots[instance],
                                rows=int(rows_per_step[step, instance]), stream=lane.stream)
            torch.cuda.synchronize()
            return time.perf_counter() - started

        run_steps((0, 1))  # warm-up
        together = run_steps((0, 1))
        alone = [run_steps((instance,)) for instance in range(2)]
        co_agent.check_health()
        colocated = {"steps": COLOCATED_STEPS, "rows_per_step": "U{1..512} per model, seed 7", "models": []}
        total_bytes = 0.0
        for instance, (c_hidden, c_inter) in enumerate(COLOCATED_SHAPES):
            rows = rows_per_step[:, instance].astype(float)
            model_bytes = float(sum(6.0 * c_hidden * c_inter + 4.0 * r * c_hidden + 4.0 * r for r in rows))
            model_flops = float(sum(6.0 * r * c_hidden * c_inter for r in rows))
            total_bytes += model_bytes
            colocated["models"].append({
                "hidden": c_hidden, "intermediate": c_inter, "tokens": int(rows.sum()),
                "tokens_per_s_concurrent": round(rows.sum() / together, 1),
                "tokens_per_s_alone": round(rows.sum() / alone[instance], 1),
                "us_per_step_alone": round(alone[instance] / COLOCATED_STEPS * 1e6, 2),
                "hbm_frac_alone": round(model_bytes / alone[instance] / 1e9 / HBM_PEAK_GBS, 4),
                "mfma_frac_alone": round(model_flops / alone[instance] / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            })
        colocated["us_per_step_concurrent"] = round(together / COLOCATED_STEPS * 1e6, 2)
        colocated["combined_hbm_frac_concurrent"] = round(total_bytes / together / 1e9 / HBM_PEAK_GBS, 4)
        co_agent.close()
        del co_pools, co_slots

    # ---------------------------------------------------------------- MoE layer
    # Qwen3-30B-A3B-shaped MoE layer (no BASELINE config names one; reported beside the
    # Dense path), registered as a MoE layer and replayed through its Lane template like a
    # Dense layer: gather + RMSNorm, Router (128 experts, softmax top-8, renormalised),
    # Experts (hidden 2048, moe_intermediate 768), combine written to the slots.  Timed with
    # HIP events on the current stream.
    def measure_moe(dtype: torch.dtype) -> dict:
        from crosspool_amd.moe import MoeFfnWeights, MoeLayerSpec, MoeRouterWeights

        m_hidden, m_inter, m_experts, m_topk = MOE_SHAPE
        generator = torch.Generator(device=device).manual_seed(18)
        moe_weights = MoeFfnWeights(
            (torch.randn((m_experts, 2 * m_inter, m_hidden), device=device, generator=generator) * 0.02).to(dtype),
            (torch.randn((m_experts, m_hidden, m_inter), device=device, generator=generator) * 0.02).to(dtype),
            MoeRouterWeights((torch.randn((m_experts, m_hidden), device=device, generator=generator) * 0.02).to(dtype)),
        )
        moe_spec = MoeLayerSpec(routed_expert_count=m_experts, routed_topk=m_topk)
        moe_agent = FfnAgent(device)
        moe_agent.register_moe_layer(instance_index=0, layer_ordinal=0, weights=moe_weights, spec=moe_spec,
                                     norm_weight=torch.ones(m_hidden, dtype=dtype, device=device))
        moe_agent.materialize(maximum_row_capacity=max(MOE_TOKENS))
        moe_pool = torch.randn((max(MOE_TOKENS) + 64, m_hidden), device=device, generator=generator).to(dtype)
        entry = {"shape": {"hidden": m_hidden, "moe_intermediate": m_inter, "experts": m_experts, "topk": m_topk},
                 "payload": str(dtype).removeprefix("torch."),
                 "execution": "MoE GraphTemplate replay (FfnAgent.register_moe_layer)", "points": []}
        for t in MOE_TOKENS:
            moe_slots = torch.arange(t, dtype=torch.int32, device=device)

            def moe_step() -> None:
                moe_agent.execute(instance_index=0, layer_ordinal=0, pool=moe_pool, slots=moe_slots,
                                  stream=torch.cuda.current_stream())

            for _ in range(3):
                moe_step()
            launches = max(10, min(100, 20000 // t))
            begin = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            begin.record()
            for _ in range(launches):
                moe_step()
            end.record()
            end.synchronize()
            moe_seconds = begin.elapsed_time(end) / 1e3 / launches
            capacity = select_capacity(derive_payload_row_capacities(max(MOE_TOKENS)), t)
            desc = moe_spec.signature(hidden_size=m_hidden, local_intermediate_size=m_inter,
                                      payload_row_capacity=capacity, payload_dtype=dtype).native_descriptor()
            ids_at = _native.moe_step_workspace_layout(desc, capacity)[4]
            ids = moe_agent.lanes[0].workspace[ids_at:ids_at + 4 * t * m_topk].view(torch.int32)
            active = int(torch.unique(ids).numel())
            flops = 2.0 * t * m_experts * m_hidden + 6.0 * t * m_topk * m_hidden * m_inter
            weight_bytes = 2.0 * m_experts * m_hidden + 6.0 * active * m_hidden * m_inter
            entry["points"].append({
                "tokens": t, "us": round(moe_seconds * 1e6, 2), "tokens_per_s": round(t / moe_seconds, 1),
                "active_experts": active,
                "hbm_frac": round((weight_bytes + 4.0 * t * m_hidden) / moe_seconds / 1e9 / HBM_PEAK_GBS, 4),
                "mfma_frac": round(flops / moe_seconds / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            })
            del moe_slots
        moe_agent.check_health()
        moe_agent.close()
        return entry

    moe = moe_fp16 = None
    if not args.no_sweep:
        moe = measure_moe(torch.bfloat16)
        moe_fp16 = measure_moe(torch.float16)

    # ---------------------------------------------------------------- fp16 Dense layer
    # The same Qwen3-8B layer with fp16 payloads (weights, norm and mailbox; the fp16
    # instantiation of every kernel), two alternating copies, at a decode and the headline
    # size.  The fp16 dense MFMA peak is the bf16 one.
    dense_fp16 = None
    if not args.no_sweep:
        half_agent = FfnAgent(device)
        for ordinal in (0, 1):
            half_agent.register_layer(
                instance_index=0, layer_ordinal=ordinal,
                weights=DenseFfnWeights.from_tensors(weights.i_proj.values.half(), weights.o_proj.values.half()),
                norm_weight=norm.half(), eps=1e-6,
            )
        half_agent.materialize(maximum_row_capacity=max_tokens)
        half_lane = half_agent.lanes[0]
        half_pool = pool.half()
        dense_fp16 = {"payload": "float16", "points": []}
        for t in (1, args.decode_tokens, args.tokens):
            def half_replay(step: int, t=t) -> None:
                half_lane.replay(instance_index=0, layer_ordinal=step % 2, pool=half_pool, slots=slots, rows=t,
                                 stream=half_lane.stream)

            for step in range(10):
                half_replay(step)
            torch.cuda.synchronize()
            steps = 2 * args.sweep_steps
            start = time.perf_counter()
            for step in range(steps):
                half_replay(step)
            torch.cuda.synchronize()
            seconds = (time.perf_counter() - start) / steps
            dense_fp16["points"].append({
                "tokens": t, "us": round(seconds * 1e6, 2), "tokens_per_s": round(t / seconds, 1),
                "hbm_frac": round(layer_bytes(t) / seconds / 1e9 / HBM_PEAK_GBS, 4),
                "mfma_frac": round(layer_flops(t) / seconds / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            })
        half_agent.check_health()
        half_agent.close()
        del half_pool

    # ---------------------------------------------------------------- ffn_shim transaction
    # Host-timed ffn_shim calls on resident [T, H] hidden states: through the Transport
    # mailbox on the caller's stream (submit -> Dense step -> settle), through it with the
    # step on the Lane's stream (two cross-stream hops), and without it.
    shim = None
    if not args.no_sweep:
        from crosspool_amd.ffn import DpRowLayout, ForwardMode, OutputRequirement
        from crosspool_amd.ops import attach, detach, ffn_shim
        from crosspool_amd.transport import FfnRequestMetadata

        metadata = FfnRequestMetadata(0, ForwardMode.DECODE, OutputRequirement.PER_RANK_COMPLETE, DpRowLayout.NONE)
        shim = {}
        for mode in ("mailbox", "mailbox_lane_stream", "direct"):
            attach(agent, mailbox=mode != "direct", lane_stream=mode == "mailbox_lane_stream")
            for t in (1, args.decode_tokens):
                x = pool[:t]
                for _ in range(10):
                    ffn_shim(x, None, metadata)
                torch.cuda.synchronize()
                calls = 3 * args.sweep_steps
                start = time.perf_counter()
                for _ in range(calls):
                    ffn_shim(x, None, metadata)
                torch.cuda.synchronize()
                shim[f"{mode}_tokens{t}_us"] = round(
                    (time.perf_counter() - start) / calls * 1e6, 2
                )
            detach()
        agent.check_health()

    # ---------------------------------------------------------------- CPU baseline
    # The oracle's torch-CPU restatement of one mailbox step (gather, RMSNorm, fp32 matmuls
    # with the reference's bf16 stage rounding, scatter) on every affinity core of the host,
    # at the headline and at each sweep point: 3 untimed runs, then the median of 10.
    cpu_baseline = None
    if not args.no_cpu_baseline:
        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)
        gate_up_f32 = w_gate_up.float()
        down_f32 = w_down.float()
        work_pool = pool_cpu.clone()

        def cpu_step(rows: int) -> None:
            index = torch.from_numpy(slots_cpu[:rows].astype("int64"))
            x = o.rmsnorm(work_pool[index], norm_weight, 1e-6)
            projected = torch.mm(x.float(), gate_up_f32.t())
            activated = o.gated_silu(projected[:, 0::2].bfloat16(), projected[:, 1::2].bfloat16())
            work_pool[index] = torch.mm(activated.float(), down_f32.t()).bfloat16()

        cpu_points = []
        for t in sorted(set(SWEEP + (tokens,))):
            for _ in range(3):
                cpu_step(t)
            durations = []
            for _ in range(10):
                started = time.perf_counter()
                cpu_step(t)
                durations.append(time.perf_counter() - started)
            median = statistics.median(durations)
            cpu_points.append({
                "tokens": t, "tokens_per_s": round(t / median, 1), "ms": round(median * 1e3, 2),
                "gbs": round(layer_bytes(t) / median / 1e9, 2), "gflops": round(layer_flops(t) / median / 1e9, 1),
            })
        headline_cpu = next(point for point in cpu_points if point["tokens"] == tokens)
        cpu_baseline = {
            "value": headline_cpu["tokens_per_s"],
            "unit": "tokens/s",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (
                f"one {tokens}-token Qwen3-8B mailbox step (gather, RMSNorm, fp32 matmuls with bf16 stage rounding, "
                f"scatter), 3 warm-up runs then the median of 10, on {threads} affinity cores of {os.cpu_count()}; "
                "weights pre-widened to fp32 outside the timing; 'points' repeats it at every sweep size"
            ),
            "points": cpu_points,
        }

    result = {
        "metric": "FFN-layer tokens/sec at Qwen3-8B shape; % HBM BW (decode) / % MFMA peak (prefill)",
        "value": round(tokens / seconds, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(seconds * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, random-init)",
        "config": {
            "workload": "qwen3-8b-ffn-layer (BASELINE config 3)",
            "hidden": HIDDEN,
            "intermediate": INTERMEDIATE,
            "tokens": tokens,
            "mailbox_slots": POOL_SLOTS,
            "rmsnorm_fused_into_gather": True,
            "execution": "GraphTemplate replay per layer signature (captured kernels launched directly)",
            "layer_mfma_frac": round(layer_flops(tokens) / seconds / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "layer_hbm_frac": round(layer_bytes(tokens) / seconds / 1e9 / HBM_PEAK_GBS, 4),
        },
        "roofline": roofline,
        "cpu_baseline": cpu_baseline,
        "decode": decode,
        "sweep": sweep,
        "tp_reduce": tp_reduce,
        "graph_dispatch": graph_dispatch,
        "shim": shim,
        "moe": moe,
        "moe_fp16": moe_fp16,
        "dense_fp16": dense_fp16,
        "config2_stack": stack,
        "config4_colocated": colocated,
        "config5_shard": shard,
    }
    agent.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
