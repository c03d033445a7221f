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
TRAFFIC_PROFILE = ROOT / "profiles" / "decode_qwen3_8b_m1_hbm_traffic.md"
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
    p.add_argument("--modes", default="grouped,grouped-fused,single,layer",
                   help="comma-separated decode launch groupings to time (first one is the headline)")
    p.add_argument("--prefill-tokens", default="64,256,512,2048",
                   help="token counts of the Llama-3-8B prefill sweep ('' to skip)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB 10 times (byte-counter calibration) and exit")
    p.add_argument("--e2e-tokens", type=int, default=128,
                   help="greedy tokens of the end-to-end decoder run (0 to skip)")
    p.add_argument("--e2e-prompt", type=int, default=512, help="prompt length of the end-to-end run")
    p.add_argument("--dominant-only", action="store_true",
                   help="only launch the dominant call (gate/up batch) of every layer eagerly --steps times "
                        "(per-dispatch counter collection) and exit")
    return p.parse_args(argv)


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


# Launch grouping per decoder layer (indices into the seven projections):
#   grouped: decode dependency order - Q/K/V share x, O, gate/up share x, down;
#   single:  one launch per linear;
#   layer:   the seven linears of a layer with independent inputs in one launch.
# A "-fused" suffix runs the same grouping with the single-kernel decode
# launch (in-kernel grid handoff) instead of the default two-kernel split.
GROUPINGS = {
    "grouped": ((0, 1, 2), (3,), (4, 5), (6,)),
    "single": ((0,), (1,), (2,), (3,), (4,), (5,), (6,)),
    "layer": ((0, 1, 2, 3, 4, 5, 6),),
}


def _grouping(mode: str):
    return GROUPINGS[mode.removesuffix("-fused")]


def build_stack(layers: int, tokens: int, device):
    """Prepared layers plus resident inputs/outputs for every linear of a step."""

    import torch

    from nanoquant_amd import synthetic as syn
    from nanoquant_amd.runtime import HipPackedBackend

    backend = HipPackedBackend()
    stack = []
    for layer in range(layers):
        shapes = syn.qwen3_8b_layer(layer)
        inputs = {}
        entries = []
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
            entries.append((shape, prepared, inputs[key], out))
        stack.append(entries)
    return backend, stack


def step_calls(stack, mode: str, backend=None):
    """The calls of one step: a list of member lists."""

    calls = [[entries[i] for i in group] for entries in stack for group in _grouping(mode)]
    if mode.endswith("-fused"):
        calls = [[(shape, backend.with_decode_launch(prepared, "fused"), x, out)
                  for shape, prepared, x, out in members] for members in calls]
    return calls


def run_step(backend, calls):
    for members in calls:
        if len(members) == 1:
            _shape, prepared, x, out = members[0]
            backend.linear_into(x, prepared, out=out)
        else:
            backend.linear_batch([m[2] for m in members], [m[1] for m in members],
                                 outs=[m[3] for m in members])


def time_mode(backend, stack, mode: str, steps: int, warmup: int, use_graph: bool) -> dict:
    """Capture one step of `mode` in a HIP graph, replay `warmup` + `steps` times;
    events bracket the timed region."""

    import torch

    calls = step_calls(stack, mode, backend)
    replay = lambda: run_step(backend, calls)  # noqa: E731
    if use_graph:
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
    for _ in range(warmup):
        replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        replay()
    stop.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - wall0) * 1e3
    ms_per_step = max(start.elapsed_time(stop), wall_ms) / steps
    tokens = calls[0][0][2].shape[0]
    step_bytes = sum(algorithmic_bytes(m[0], tokens) for members in calls for m in members)
    call_ms = ms_per_step / len(calls)
    return {
        "ms_per_step": ms_per_step,
        "calls_per_step": len(calls),
        "kernels_per_step": len(calls) * (1 if mode.endswith("-fused") else 2),
        "step_bytes": step_bytes,
        "mean_call_us": call_ms * 1e3,
        "bytes_per_call": step_bytes / len(calls),
        "achieved_gbs": step_bytes / len(calls) / (call_ms * 1e-3) / 1e9,
    }


# The dominant decode call: the gate/up batch (two 4096 -> 12288 linears that
# share x), the largest byte count of any call in a decode step.
DOMINANT_GROUP = (4, 5)


def time_dominant_call(backend, stack, steps: int, warmup: int) -> dict:
    """Mean duration of the dominant call (gate/up batch, k_decode_stage1 +
    k_decode_stage2) over the stack's distinct layers, captured in one HIP
    graph and bracketed by events recorded on the stream the graph runs on."""

    import torch

    calls = [[entries[i] for i in DOMINANT_GROUP] for entries in stack]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run_step(backend, calls)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            run_step(backend, calls)
        for _ in range(warmup):
            graph.replay()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(side)
        for _ in range(steps):
            graph.replay()
        stop.record(side)
    stop.synchronize()
    tokens = calls[0][0][2].shape[0]
    call_us = start.elapsed_time(stop) * 1e3 / (steps * len(calls))
    call_bytes = sum(algorithmic_bytes(m[0], tokens) for m in calls[0])
    return {"mean_call_us": call_us, "bytes_per_call": call_bytes,
            "achieved_gbs": call_bytes / (call_us * 1e-6) / 1e9, "calls": len(calls)}


def measured_traffic(tokens: int, layers: int):
    """HBM bytes per dominant call from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (calibrated against a plain copy), when it was measured
    on this exact workload; None otherwise. Counters cannot be read inside a
    timed run."""

    import re

    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_call = (\d+) \(call gate/up, tokens (\d+), layers (\d+)\)", text)
    if not m or (int(m.group(2)), int(m.group(3))) != (tokens, layers):
        return None
    return int(m.group(1))


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
        "value": round(tokens / (median * layers), 4),
        "unit": "tok/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (
            f"oracle torch fp32 forward (unpack once, 2x F.linear) over the 7 Qwen3-8B linears "
            f"of one layer at M={tokens}, {len(samples)} timed reps (median "
            f"{median * 1e3:.1f} ms/layer), scaled x{layers} layers; cpu={_cpu_model()}"
        ),
    }


FP16_DENSE_PEAK_TFLOPS = 2500.0


def prefill_sweep(token_counts, steps: int, warmup: int) -> dict:
    """Config: the seven Llama-3-8B linears (~0.8 bpw) at each token count, one
    layer pass (every linear once) captured in a HIP graph so host launch costs
    stay out of the timing; events bracket `steps` replays. TFLOP/s counts the
    two sign GEMMs (2*M*(in*r + r*out)) against the fp16 dense MFMA peak."""

    import torch

    from nanoquant_amd import synthetic as syn
    from nanoquant_amd.runtime import HipPackedBackend

    device = torch.device("cuda", 0)
    backend = HipPackedBackend()
    shapes = syn.llama3_8b_layer()
    layers = [backend.prepare(syn.synthetic_packed_layer(s, seed=syn.BASE_SEED + 500 + i, device=device), device)
              for i, s in enumerate(shapes)]
    sweep = {}
    for tokens in token_counts:
        xs = {s.in_features: syn.synthetic_activations(tokens, s.in_features, seed=tokens, device=device)
              for s in shapes}
        outs = [torch.empty(tokens, s.out_features, dtype=torch.float32, device=device) for s in shapes]

        def layer_pass():
            for s, layer, out in zip(shapes, layers, outs):
                backend.linear_into(xs[s.in_features], layer, out=out)

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            layer_pass()  # allocates the calls' workspaces outside the capture
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                layer_pass()
            for _ in range(warmup):
                graph.replay()
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(side)
            for _ in range(steps):
                graph.replay()
            stop.record(side)
        stop.synchronize()
        ms = start.elapsed_time(stop) / steps
        flops = sum(2 * tokens * (s.in_features * s.rank + s.rank * s.out_features) for s in shapes)
        tflops = flops / (ms * 1e-3) / 1e12
        sweep[str(tokens)] = {
            "ms_per_layer": round(ms, 4),
            "tok_per_s": round(tokens * 1000.0 / ms, 1),
            "tflops": round(tflops, 2),
            "frac_of_fp16_peak": round(tflops / FP16_DENSE_PEAK_TFLOPS, 4),
        }
    return {
        "workload": "llama-3-8b-shape packed linears (q/o r1638, k/v r655, gate/up/down r2549), one layer",
        "peak_tflops": FP16_DENSE_PEAK_TFLOPS,
        "points": sweep,
    }


def e2e_decode(layers: int, prompt_len: int, new_tokens: int, repeats: int, packed_us_per_layer: float) -> dict:
    """Greedy decode of a random-init Qwen3-8B-shaped model (36 layers, hidden
    4096, intermediate 12288, GQA 32/8 x 128, vocab 151936; every projection
    packed at ~1.0 bpw, bf16 N(0, 0.02) embeddings and untied lm_head, bf16
    KV cache): a `prompt_len`-token prompt through the prefill path, then
    `new_tokens` greedy tokens, each decode step one HIP-graph replay. Events
    bracket prefill and decode; the best of `repeats` runs is reported."""

    import torch

    from nanoquant_amd import synthetic as syn
    from nanoquant_amd.runtime.decoder_shell import DecoderShellConfig, PackedDecoder

    device = torch.device("cuda", 0)
    config = DecoderShellConfig(layers=layers)
    weights = syn.synthetic_decoder(config, seed=syn.BASE_SEED + 5, device=device)
    decoder = PackedDecoder(config, weights, device=device, max_positions=prompt_len + new_tokens)
    del weights
    g = torch.Generator().manual_seed(syn.BASE_SEED + 5)
    prompt = torch.randint(0, config.vocab, (prompt_len,), generator=g).to(device)
    decoder.generate_greedy(prompt, new_tokens)  # capture + warm-up
    runs = []
    tokens = None
    for _ in range(repeats):
        timing: dict = {}
        out = decoder.generate_greedy(prompt, new_tokens, timings=timing)
        if tokens is None:
            tokens = out.tolist()
        elif out.tolist() != tokens:
            raise RuntimeError("end-to-end greedy decode is not deterministic across runs")
        runs.append(timing)
    best = min(runs, key=lambda r: r["decode_ms"])
    decode_steps = new_tokens - 1
    ms_per_token = best["decode_ms"] / decode_steps
    # per layer: unfused RMSNorm, QKV (2), attention (2), O (2), RMSNorm, gate/up (2), SiLU product,
    # down (2); fused: the two norms and the SiLU product run inside the packed calls (layer 0 keeps
    # its input norm). Plus embedding, final norm, lm_head and greedy select.
    kernels = layers * 10 + 5 if decoder.fuse_decode else layers * 12 + 4
    return {
        "workload": (f"qwen3-8b-shape random-init packed model, {layers} layers, vocab {config.vocab}, "
                     f"prompt {prompt_len} ids, {new_tokens} greedy tokens, batch 1, bf16 activations/KV"),
        "decode_tok_per_s": round(1000.0 / ms_per_token, 2),
        "decode_ms_per_token": round(ms_per_token, 4),
        "prefill_ms": round(best["prefill_ms"], 3),
        "prefill_tok_per_s": round(prompt_len * 1000.0 / best["prefill_ms"], 1),
        "total_tok_per_s": round(new_tokens * 1000.0 / (best["prefill_ms"] + best["decode_ms"]), 2),
        "packed_linear_us_per_layer": round(packed_us_per_layer, 2),
        "shell_us_per_token": round(ms_per_token * 1000.0 - packed_us_per_layer * layers, 1),
        "kernels_per_token": kernels,
        "fused_decode": decoder.fuse_decode,
        "first_tokens": tokens[:8],
        "repeats": repeats,
    }


def copy_calibration(mib: int) -> int:
    """A plain device-to-device copy of known size, for scaling HBM byte counters."""

    import torch

    src = torch.ones(mib * (1 << 20) // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": src.numel() * 4, "written": dst.numel() * 4}))
    return 0


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

    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    modes_wanted = [m for m in args.modes.split(",") if m]
    if not modes_wanted or any(m.removesuffix("-fused") not in GROUPINGS for m in modes_wanted):
        print(f"--modes must name some of {sorted(GROUPINGS)} (optionally with -fused)", file=sys.stderr)
        return 2

    import torch

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    print(f"[bench] building {args.layers}-layer stack, M={args.tokens}", file=sys.stderr, flush=True)
    backend, stack = build_stack(args.layers, args.tokens, device)
    torch.cuda.synchronize()
    if args.dominant_only:
        calls = [[entries[i] for i in DOMINANT_GROUP] for entries in stack]
        for _ in range(args.steps):
            run_step(backend, calls)
        torch.cuda.synchronize()
        print(json.dumps({"dominant_calls": args.steps * len(calls),
                          "bytes_per_call": sum(algorithmic_bytes(m[0], args.tokens) for m in calls[0])}))
        return 0
    modes = {}
    for mode in modes_wanted:
        print(f"[bench] mode {mode}: timing {args.steps} steps", file=sys.stderr, flush=True)
        modes[mode] = time_mode(backend, stack, mode, args.steps, args.warmup, not args.no_graph)
    head_mode = modes_wanted[0]
    head = modes[head_mode]
    ms_per_step = head["ms_per_step"]
    print("[bench] dominant call (gate/up batch) timing", file=sys.stderr, flush=True)
    dom = time_dominant_call(backend, stack, args.steps, args.warmup)
    achieved = dom["achieved_gbs"]

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
                f"(q/o r2048, k/v r819, gate/up/down r3072), M={args.tokens}, one HIP-graph step, "
                f"launch grouping '{head_mode}'"
            ),
            "global_batch": args.tokens,
            "layers": args.layers,
            "linears_per_step": 7 * args.layers,
            "weight_bytes_per_step": sum(e[0].weight_bytes for entries in stack for e in entries),
            "parallelism": "single-gpu",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(args.tokens, args.layers),
            "traffic_source": TRAFFIC_PROFILE.name,
            "kernel": ("dominant decode call: gate/up batch (two 4096->12288 r3072 linears sharing x) = "
                       "k_decode_stage1 + k_decode_stage2, graph of one call per layer"),
            "bytes_per_call": round(dom["bytes_per_call"]),
            "mean_call_us": round(dom["mean_call_us"], 3),
            "step_achieved_gbs": round(head["achieved_gbs"], 1),
        },
        "calls_per_step": head["calls_per_step"],
        "kernels_per_step": head["kernels_per_step"],
        "modes": {
            name: {
                "calls_per_step": m["calls_per_step"],
                "kernels_per_step": m["kernels_per_step"],
                "ms_per_step": round(m["ms_per_step"], 4),
                "tok_per_s": round(args.tokens * 1000.0 / m["ms_per_step"], 2),
                "mean_call_us": round(m["mean_call_us"], 3),
                "bytes_per_call": round(m["bytes_per_call"]),
                "achieved_gbs": round(m["achieved_gbs"], 1),
                "frac_of_hbm_peak": round(m["achieved_gbs"] / HBM_PEAK_GBS, 4),
            }
            for name, m in modes.items()
        },
        "prefill": None,
        "cpu_baseline": None,
    }
    prefill_tokens = [int(t) for t in args.prefill_tokens.split(",") if t]
    if prefill_tokens:
        print(f"[bench] prefill sweep M={prefill_tokens}", file=sys.stderr, flush=True)
        result["prefill"] = prefill_sweep(prefill_tokens, max(args.steps // 2, 3), 2)
    if args.e2e_tokens > 0:
        print(f"[bench] end-to-end decode: prompt {args.e2e_prompt}, {args.e2e_tokens} tokens",
              file=sys.stderr, flush=True)
        packed_us = modes["grouped"]["ms_per_step"] * 1000.0 / args.layers if "grouped" in modes else float("nan")
        result["e2e"] = e2e_decode(args.layers, args.e2e_prompt, args.e2e_tokens, 3, packed_us)
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(args.tokens, args.cpu_seconds, args.layers)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
