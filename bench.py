"""Benchmark: exact attention of one MiniMax-H3 denoise step on one MI355X.

Workload (one "step"): 50 attention layers of dense non-causal bf16 attention,
B=1, H=56, S=42120 (packed text 512 + cond 256 + audio 2048 + video 39304),
D=128, fresh seeded synthetic inputs per layer (q,k ~ N(0,1), v ~ 4 N(0,1)),
all resident in HBM before timing starts.  Metric: attention TFLOP/s
(4*S^2*D*H per layer) and % of the dense bf16 MFMA peak; ms per 50-layer step.

Prints ONE JSON line.  Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "minimaxh3-on-a100-x4_amd"))

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA: 256 CU x 4096 FLOP/clk x 2.4 GHz
# HBM bytes per launch of the dense kernel at this shape, from the rocprofv3
# FETCH_SIZE (x2.0) and WRITE_SIZE (x1.0) passes recorded in
# profiles/attn_dense_h56_s42120_counters.txt (scales from a 2048 MiB copy).
MEASURED_TRAFFIC_BYTES = 8.632e9
B, H, S, D, LAYERS = 1, 56, 42120, 128, 50


def flops_per_layer(h=H, s=S, d=D):
    return 4.0 * s * s * d * h


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(budget_s: float = 12.0):
    """The reference's attention call (torch SDPA, attn_sm80/attn_sm80.py:33-35 and
    harness/sp_runtime.py:119-121) on bf16 CPU tensors, on a head subset at full S,
    extrapolated linearly in H (heads are independent)."""
    import torch
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    hs = 1
    q, k, v = (torch.randn(1, hs, S, D, generator=g).to(torch.bfloat16) for _ in range(3))
    torch.nn.functional.scaled_dot_product_attention(q[:, :, :512], k, v)  # warm-up
    t0 = time.perf_counter()
    torch.nn.functional.scaled_dot_product_attention(q, k, v)
    per_head = time.perf_counter() - t0
    reps = max(1, min(8, int(budget_s / max(per_head, 1e-3)) - 1))
    t0 = time.perf_counter()
    for _ in range(reps):
        torch.nn.functional.scaled_dot_product_attention(q, k, v)
    per_head = (time.perf_counter() - t0) / reps
    layer_s = per_head * H
    return {
        "value": round(flops_per_layer() / layer_s / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "reference",
        "sample": (f"torch SDPA (CPU, bf16) on {hs} head x {reps} reps at S={S}, D={D}; "
                   f"{per_head * 1e3:.0f} ms/head, extrapolated x{H} heads = "
                   f"{layer_s:.2f} s/layer, {layer_s * LAYERS:.0f} s per 50-layer step; "
                   f"CPU: {cpu_model()}"),
        "ms_per_layer": round(layer_s * 1e3, 1),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the timed region, run one device copy of this many MiB "
                         "(reference kernel for scaling FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported "
              "(the attention path is single-GPU; see DESIGN.md for how it shards)", file=sys.stderr)
        sys.exit(2)

    import torch
    import h3attn

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = args.layers
    qs, ks, vs = [], [], []
    for layer in range(L):
        g = torch.Generator(device=dev).manual_seed(1000 + layer)
        qs.append(torch.randn(B, H, S, D, generator=g, device=dev, dtype=torch.bfloat16))
        ks.append(torch.randn(B, H, S, D, generator=g, device=dev, dtype=torch.bfloat16))
        vs.append(torch.randn(B, H, S, D, generator=g, device=dev, dtype=torch.bfloat16).mul_(4))
    out = torch.empty(B, H, S, D, device=dev, dtype=torch.bfloat16)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)

    def step(events=None):
        for layer in range(L):
            if events is not None:
                events[layer][0].record(stream)
            h3attn.attn_fwd(qs[layer], ks[layer], vs[layer], out=out)
            if events is not None:
                events[layer][1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region: exactly `steps` steps, synchronised on both sides.  HIP events
    # bracket every launch on the launch stream for the per-kernel average.
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(L)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step(evs[s])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    if args.calib_copy_mib > 0:
        src = torch.empty(args.calib_copy_mib << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    kern_ms = [a.elapsed_time(b) for st in evs for a, b in st]
    avg_kernel_ms = sum(kern_ms) / len(kern_ms)
    ms_per_step = wall * 1e3 / args.steps
    total_flops = flops_per_layer() * L * args.steps
    value = total_flops / wall / 1e12
    achieved = flops_per_layer() / (avg_kernel_ms * 1e-3) / 1e12

    res = {
        "metric": "attn TFLOP/s & % bf16 MFMA peak at H=56,S=42120,D=128; ms per 50-layer step",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded device RNG, fresh q/k/v per layer, resident in HBM)",
        "config": {"workload": f"dense exact non-causal attention, {L} layers per step",
                   "B": B, "H": H, "S": S, "D": D, "layers": L,
                   "segments": "text 512 + cond 256 + audio 2048 + video 39304"},
        "pct_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "ms_per_layer": round(avg_kernel_ms, 3),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": MEASURED_TRAFFIC_BYTES, "kernel": "attn_fwd_kernel<8,false>",
                     "flop_per_launch": flops_per_layer(),
                     "avg_launch_ms": round(avg_kernel_ms, 3)},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
