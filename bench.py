"""FFN-layer throughput of the MI355X FfnAgent path at the Qwen3-8B shape.

One step = one replay of the Dense mailbox step's GraphTemplate (its captured
kernels launched on the Lane stream) for a batch of T tokens: gather T seeded slots of an 8192-slot bf16 mailbox with the fused
RMSNorm, gate_up [4096 -> 2 x 12288] + SiLU*mul, down [12288 -> 4096],
scatter back into the same slots.  Inputs are resident in HBM before timing.

Prints ONE JSON line: the headline at T = --tokens (default 2048, the
MFMA-bound north-star point), a ``decode`` entry at T = 32 (HBM-bound), the
batch sweep of BASELINE config 3, the roofline of the dominant kernel
(measured with HIP events on the Lane stream it runs on) and the CPU
baseline (the oracle's torch-CPU restatement on the host cores).

``--kernels-only`` instead launches just the kernels whose hardware counters
the roofline's ``traffic`` figure comes from (a byte copy of known size for
calibration, then gate_up at the headline and decode sizes), for
``rocprofv3 --pmc`` runs; ``profiles/traffic.json`` records their result.
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
    parser.add_argument("--cpu-seconds", type=float, default=10.0, help="bounded CPU-baseline sample length")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--kernels-only", action="store_true", help="launch only the profiled kernels, then exit")
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
    from crosspool_amd.weights import DenseFfnWeights
    from oracle import ffn_oracle as o

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
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
    agent.materialize(maximum_row_capacity=max_tokens)
    lane = agent.lanes[0]
    torch.cuda.synchronize()

    def replay(tokens: int) -> None:
        lane.replay(instance_index=0, layer_ordinal=0, pool=pool, slots=slots, rows=tokens, stream=lane.stream)

    def time_replays(tokens: int, steps: int, warmup: int) -> float:
        for _ in range(warmup):
            replay(tokens)
        torch.cuda.synchronize()
        start = time.perf_counter()
        for _ in range(steps):
            replay(tokens)
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
            return {
                "kernel": variant, "tokens": tokens, "bound": "mfma", "achieved": round(achieved, 1),
                "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                "traffic": traffic, "avg_launch_us": round(per_launch * 1e6, 2),
                "algorithmic_flops": gate_up_flops(tokens),
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
        for t in (tokens, args.decode_tokens):
            gate_up_launches(t, 6)
        torch.cuda.synchronize()
        agent.close()
        print(json.dumps({"kernels_only": True, "copy_bytes": CALIBRATION_COPY_BYTES,
                          "gate_up_tokens": [tokens, args.decode_tokens]}), flush=True)
        return 0

    # ---------------------------------------------------------------- headline
    seconds = time_replays(tokens, args.steps, args.warmup)
    agent.check_health()
    roofline = kernel_roofline(tokens, max(20, min(args.steps, 200)))

    # ---------------------------------------------------------------- decode point
    decode_seconds = time_replays(args.decode_tokens, args.steps, args.warmup)
    decode = {
        "tokens": args.decode_tokens,
        "tokens_per_s": round(args.decode_tokens / decode_seconds, 1),
        "us_per_layer": round(decode_seconds * 1e6, 2),
        "layer_hbm_frac": round(layer_bytes(args.decode_tokens) / decode_seconds / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": kernel_roofline(args.decode_tokens, 200),
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

    # ---------------------------------------------------------------- MoE layer
    # Qwen3-30B-A3B-shaped MoE layer (no BASELINE config names one; reported beside the
    # Dense path): Router (128 experts, softmax top-8, renormalised) + Experts (hidden 2048,
    # moe_intermediate 768), timed with HIP events on the current stream.
    moe = None
    if not args.no_sweep:
        from crosspool_amd.moe import Experts, MoeFfnWeights, MoeRouterWeights, Router

        m_hidden, m_inter, m_experts, m_topk = MOE_SHAPE
        generator = torch.Generator(device=device).manual_seed(18)
        moe_weights = MoeFfnWeights(
            (torch.randn((m_experts, 2 * m_inter, m_hidden), device=device, generator=generator) * 0.02).bfloat16(),
            (torch.randn((m_experts, m_hidden, m_inter), device=device, generator=generator) * 0.02).bfloat16(),
        )
        router_weights = MoeRouterWeights(
            (torch.randn((m_experts, m_hidden), device=device, generator=generator) * 0.02).bfloat16()
        )
        moe = {"shape": {"hidden": m_hidden, "moe_intermediate": m_inter, "experts": m_experts, "topk": m_topk},
               "points": []}
        for t in MOE_TOKENS:
            x = torch.randn((t, m_hidden), device=device, generator=generator).bfloat16()
            router = Router(row_capacity=t, hidden_size=m_hidden, routed_expert_count=m_experts, routed_topk=m_topk,
                            device=device)
            experts_op = Experts(row_capacity=t, hidden_size=m_hidden, local_intermediate_size=m_inter,
                                 expert_count=m_experts, effective_topk=m_topk, device=device)
            out = torch.empty_like(x)

            def moe_step() -> None:
                router.run_into(hidden_states=x, router_weights=router_weights)
                experts_op.run_into(hidden_states=x, weights=moe_weights, topk_ids=router.ids,
                                    topk_weights=router.weights, output=out)

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
            active = int(torch.unique(router.ids).numel())
            flops = 2.0 * t * m_experts * m_hidden + 6.0 * t * m_topk * m_hidden * m_inter
            weight_bytes = 2.0 * m_experts * m_hidden + 6.0 * active * m_hidden * m_inter
            moe["points"].append({
                "tokens": t, "us": round(moe_seconds * 1e6, 2), "tokens_per_s": round(t / moe_seconds, 1),
                "active_experts": active,
                "hbm_frac": round((weight_bytes + 4.0 * t * m_hidden) / moe_seconds / 1e9 / HBM_PEAK_GBS, 4),
                "mfma_frac": round(flops / moe_seconds / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            })
            del router, experts_op, x, out
        del moe_weights, router_weights
        agent.check_health()

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
    cpu_baseline = None
    if not args.no_cpu_baseline:
        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)
        sample_tokens = 256
        gate_up_f32 = w_gate_up.float()
        down_f32 = w_down.float()
        sample_slots = slots_cpu[:sample_tokens]
        work_pool = pool_cpu.clone()

        def cpu_step() -> None:
            x = o.rmsnorm(o.gather(work_pool, sample_slots), norm_weight, 1e-6)
            projected = torch.mm(x.float(), gate_up_f32.t())
            activated = o.gated_silu(projected[:, 0::2].bfloat16(), projected[:, 1::2].bfloat16())
            y = torch.mm(activated.float(), down_f32.t()).bfloat16()
            o.scatter(work_pool, sample_slots, y)

        for _ in range(2):
            cpu_step()
        durations = []
        deadline = time.perf_counter() + args.cpu_seconds
        while len(durations) < 3 or time.perf_counter() < deadline:
            started = time.perf_counter()
            cpu_step()
            durations.append(time.perf_counter() - started)
        median = statistics.median(durations)
        cpu_baseline = {
            "value": round(sample_tokens / median, 1),
            "unit": "tokens/s",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (
                f"{len(durations)} runs of one {sample_tokens}-token Qwen3-8B mailbox step (gather, RMSNorm, fp32 "
                f"matmuls with bf16 stage rounding, scatter) on {threads} affinity cores of {os.cpu_count()}; "
                "median; weights pre-widened to fp32 outside the timing"
            ),
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
        "shim": shim,
        "moe": moe,
        "config2_stack": stack,
    }
    agent.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
