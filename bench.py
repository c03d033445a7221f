#!/usr/bin/env python
"""Decode throughput of a Qwen3-8B-shaped packed-linear stack on one MI355X.

Workload (one "step" = one decode token through every packed linear of the
model): 36 decoder layers x 7 packed binary low-rank linears at ~1.0 bpw
(q/o 4096->4096 r2048, k/v 4096->1024 r819, gate/up 4096->12288 r3072,
down 12288->4096 r3072), 874.9 MB of distinct packed weights (well above the
256 MB Infinity Cache), synthetic Bernoulli(0.5) signs, fp16 lognormal scales,
bf16 N(0,1) activations resident in HBM, fp32 outputs (the backend boundary).
The step is captured once in a HIP graph and replayed.

Prints one JSON line (metric/value/unit, ms_per_step, roofline, cpu_baseline).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "decode tok/s (Qwen3-8B-shape, ~1bpw); packed GEMV HBM GB/s vs peak"


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--layers", type=int, default=36)
    p.add_argument("--tokens", type=int, default=1, help="decode token slots per step (1-16)")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-baseline time budget")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-graph", action="store_true", help="time eager launches instead of a graph")
    return p.parse_args(argv)


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def build_stack(layers: int, tokens: int, device):
    """Prepared layers plus resident inputs/outputs for every linear call of a step."""

    import torch

    from nanoquant_amd import synthetic as syn
    from nanoquant_amd.runtime import HipPackedBackend

    backend = HipPackedBackend()
    calls = []
    for layer in range(layers):
        shapes = syn.qwen3_8b_layer(layer)
        inputs = {}
        for i, shape in enumerate(shapes):
            state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + 1000 * layer + i, device=device)
            prepared = backend.prepare(state, device)
            role = shape.name.split(".")[-1]
            key = {"q_proj": "attn", "k_proj": "attn", "v_proj": "attn", "o_proj": "o",
                   "gate_proj": "mlp", "up_proj": "mlp", "down_proj": "down"}[role]
            if key not in inputs:
                inputs[key] = syn.synthetic_activations(
                    tokens, shape.in_features, seed=layer * 10 + i, device=device)
            out = torch.empty(tokens, shape.out_features, dtype=torch.float32, device=device)
            calls.append((shape, prepared, inputs[key], out))
    return backend, calls


def run_step(backend, calls):
    for _shape, prepared, x, out in calls:
        backend.linear_into(x, prepared, out=out)


def algorithmic_bytes(shape, tokens: int) -> int:
    """Sign words + fp16 scales + bf16 x + fp32 y (the rank-r latent is excluded)."""

    return shape.weight_bytes + 2 * tokens * shape.in_features + 4 * tokens * shape.out_features


def cpu_baseline(tokens: int, budget_s: float, layers: int) -> dict:
    """The oracle's restatement of the reference CPU torch path (unpack once, two
    fp32 F.linear per linear) on the 7 linears of one layer, scaled to the stack."""

    import torch

    from nanoquant_amd import synthetic as syn
    from oracle import nq_oracle as orc

    forwards, inputs = [], []
    for i, shape in enumerate(syn.qwen3_8b_layer(0)):
        state = syn.synthetic_packed_layer(shape, seed=syn.BASE_SEED + i)
        forwards.append(orc.CpuPackedForward(orc.operands_from_state(state)))
        inputs.append(syn.synthetic_activations(tokens, shape.in_features, seed=i))

    def one_layer():
        for fwd, x in zip(forwards, inputs):
            fwd(x)

    one_layer()
    samples = []
    begin = time.perf_counter()
    while (time.perf_counter() - begin < budget_s and len(samples) < 200) or len(samples) < 3:
        t0 = time.perf_counter()
        one_layer()
        samples.append(time.perf_counter() - t0)
    samples.sort()
    median = samples[len(samples) // 2]
    return {
        "value": tokens / (median * layers),
        "unit": "tok/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (
            f"oracle torch fp32 forward (unpack once, 2x F.linear) over the 7 Qwen3-8B linears "
            f"of one layer at M={tokens}, {len(samples)} timed reps (median "
            f"{median * 1e3:.1f} ms/layer), scaled x{layers} layers; cpu={_cpu_model()}"
        ),
    }


def main(argv=None) -> int:
    args = parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
            "multi-GPU runs are not part of this build",
            file=sys.stderr,
        )
        return 2
    if not 1 <= args.tokens <= 16:
        print("--tokens must be in 1..16 (decode path)", file=sys.stderr)
        return 2

    import torch

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    print(f"[bench] building {args.layers}-layer stack, M={args.tokens}", file=sys.stderr, flush=True)
    backend, calls = build_stack(args.layers, args.tokens, device)
    torch.cuda.synchronize()
    step_bytes = sum(algorithmic_bytes(shape, args.tokens) for shape, *_ in calls)

    # Capture the step once (outputs/workspaces live in the graph's pool).
    replay = lambda: run_step(backend, calls)  # noqa: E731
    graph = None
    if not args.no_graph:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run_step(backend, calls)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run_step(backend, calls)
        replay = graph.replay

    for _ in range(args.warmup):
        replay()
    torch.cuda.synchronize()
    print(f"[bench] warmup done; timing {args.steps} steps", file=sys.stderr, flush=True)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        replay()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    gpu_ms = start.elapsed_time(stop)
    ms_per_step = max(gpu_ms, wall * 1e3) / args.steps

    # Every launch inside the timed graph is the fused decode kernel (outputs and
    # workspaces are preallocated in the graph pool), so the event-timed region
    # divided by the launch count is its average launch duration, inter-kernel
    # gaps included.
    launches = args.steps * len(calls)
    mean_launch_ms = ms_per_step * args.steps / launches
    mean_bytes = step_bytes / len(calls)
    achieved = mean_bytes / (mean_launch_ms * 1e-3) / 1e9

    result = {
        "metric": METRIC,
        "value": round(args.tokens * 1000.0 / ms_per_step, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16-in/fp32-acc (1-bit signs)",
        "data": "synthetic (Bernoulli(0.5) signs, fp16 lognormal(0,0.25) scales, bf16 N(0,1) x)",
        "config": {
            "workload": (
                f"qwen3-8b-shape packed-linear decode stack: {args.layers} layers x 7 linears "
                f"(q/o r2048, k/v r819, gate/up/down r3072), M={args.tokens}, HIP-graph step"
            ),
            "global_batch": args.tokens,
            "layers": args.layers,
            "linears_per_step": len(calls),
            "weight_bytes_per_step": sum(s.weight_bytes for s, *_ in calls),
            "parallelism": "single-gpu",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "k_decode_fused (one launch per packed linear)",
            "bytes_per_launch": round(mean_bytes),
            "mean_launch_us": round(mean_launch_ms * 1e3, 3),
        },
        "launches_per_step": len(calls),
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(args.tokens, args.cpu_seconds, args.layers)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
