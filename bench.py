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
NOMINAL_CLOCK_GHZ = 2.4
FLOP_PER_CLK = 256 * 4096  # dense bf16 MFMA, whole chip
# HBM bytes per launch of the dense kernel at this shape come from the rocprofv3
# FETCH_SIZE (x2.0) and WRITE_SIZE (x1.0) passes summarised in this file (each
# counter scaled by what it reads for a 2048 MiB device copy); its line
# "roofline.traffic = <bytes> B" is read at run time.
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "attn_dense_h56_s42120_counters.txt")
SPARSE_TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "attn_sparse_h56_s42120_counters.txt")
TILES_TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "attn_tiles_h56_s42120_counters.txt")
PROLOGUE_TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "prologue_s8192_h56.txt")
B, H, S, D, LAYERS = 1, 56, 42120, 128, 50


def measured_traffic(path=TRAFFIC_SUMMARY, key=""):
    """(bytes per launch, source) from a committed counter summary's "roofline.traffic[.key] = X B"
    line, or (None, reason)."""
    import re
    pat = r"\s*roofline\.traffic" + (r"\." + re.escape(key) if key else "") + r"\s*=\s*([0-9.]+[eE][+]?[0-9]+)\s*B\b"
    try:
        with open(path) as f:
            for ln in f:
                m = re.match(pat, ln)
                if m:
                    return float(m.group(1)), os.path.relpath(path, ROOT)
    except OSError as e:
        return None, f"unreadable: {e}"
    return None, "no roofline.traffic line"


def _clock_from_rows(rows):
    ghz = [r[7] / (r[8] * 10.0) for r in rows if r[8] > 0]
    return (sum(ghz) / len(ghz), min(ghz), max(ghz)) if ghz else None


def measure_clock_sparse(item, blk, tiles=False):
    """As measure_clock, for the block-sparse kernel: one profiled launch of the first
    layer's inputs (the ping-pong sparse kernels record workgroup 0's phases); `tiles`:
    the item holds a tile LUT."""
    from h3attn import ops
    try:
        q, k, v, lut, cnt, _ = item
        out = torch_empty_like(q)

        def run():
            if tiles:
                ops.attn_fwd_blocksparse_tiles_profiled(q, k, v, lut, cnt, out=out)
            else:
                ops.attn_fwd_blocksparse_profiled(q, k, v, lut, cnt, blk, blk, out=out)
        run()
        ops.prof_reset()
        run()
        c = _clock_from_rows(ops.prof_read())
        if c is None:
            return None, "no profile rows"
        return c[0], (f"s_memtime / s_memrealtime over workgroup 0's stage loop, one profiled layer after the "
                      f"timed steps; waves {c[1]:.3f}-{c[2]:.3f} GHz")
    except (RuntimeError, ValueError) as e:
        return None, f"not measured: {e}"


def torch_empty_like(t):
    import torch
    return torch.empty_like(t)


def measure_clock(torch, h3attn, dev, heads=H):
    """Shader clock under this workload, measured in this process: one dense layer of the
    same shape through the phase-profile build, whose workgroup 0 counts shader-clock
    ticks (s_memtime) and 100 MHz ticks (s_memrealtime) over its stage loop.  Returns
    (GHz averaged over the workgroup's 8 waves, note) or (None, reason)."""
    from h3attn import ops
    try:
        if not ops.prof_enabled(profile=True):
            return None, "profile build records nothing"
        g = torch.Generator(device=dev).manual_seed(77)
        q, k, v = (torch.randn(B, heads, S, D, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(3))
        out = torch.empty_like(q)
        ops.attn_fwd_profiled(q, k, v, out=out)  # warm: the clock settles under load
        ops.prof_reset()
        ops.attn_fwd_profiled(q, k, v, out=out)
        c = _clock_from_rows(ops.prof_read())
        del q, k, v, out
        if c is None:
            return None, "no profile rows"
        return c[0], (f"s_memtime / s_memrealtime over workgroup 0's stage loop, one profiled "
                      f"layer (H={heads}, S={S}) after the timed steps; waves {c[1]:.3f}-{c[2]:.3f} GHz")
    except (RuntimeError, ValueError) as e:
        return None, f"not measured: {e}"


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


def cpu_baseline(budget_s: float = 12.0, heads: int = H):
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
    layer_s = per_head * heads
    return {
        "value": round(flops_per_layer(h=heads) / layer_s / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "reference",
        "sample": (f"torch SDPA (CPU, bf16) on {hs} head x {reps} reps at S={S}, D={D}; "
                   f"{per_head * 1e3:.0f} ms/head, extrapolated x{heads} heads = "
                   f"{layer_s:.2f} s/layer, {layer_s * LAYERS:.0f} s per 50-layer step; "
                   f"CPU: {cpu_model()}"),
        "ms_per_layer": round(layer_s * 1e3, 1),
    }


def cpu_config1(torch, reps: int = 5):
    """The CPU-runnable dense case (B=1, H=4, S=2048, D=128, bf16, N(0,1) from a seed) timed
    with torch SDPA on the host cores: the MATH backend and the default CPU flash backend."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 4, 2048, D, generator=g).to(torch.bfloat16) for _ in range(3))
    fl = flops_per_layer(h=4, s=2048)
    out = {"shape": "B=1 H=4 S=2048 D=128 bf16", "cores": torch.get_num_threads()}
    for name, backends in (("math", [SDPBackend.MATH]), ("flash", [SDPBackend.FLASH_ATTENTION])):
        try:
            with sdpa_kernel(backends):
                torch.nn.functional.scaled_dot_product_attention(q, k, v)
                t0 = time.perf_counter()
                for _ in range(reps):
                    torch.nn.functional.scaled_dot_product_attention(q, k, v)
                dt = (time.perf_counter() - t0) / reps
            out[f"{name}_ms"] = round(dt * 1e3, 2)
            out[f"{name}_tflops"] = round(fl / dt / 1e12, 4)
        except RuntimeError as e:
            out[f"{name}_ms"] = None
            out[f"{name}_error"] = str(e)[:120]
    return out


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--workload", default="dense",
                    choices=["dense", "h14", "sparse", "prologue", "fused", "graph"],
                    help="dense: the headline (H=56, S=42120, 50 layers); h14: one GPU's share of "
                         "4-way head parallelism (H=14); sparse: block-sparse top-25%%+diagonal at "
                         "128x128 tiles; prologue: qk-RMSNorm+RoPE at S=8192, H=56 (GB/s); fused: "
                         "prologue + attention on the fused QKV layout at S=8192, H=56; graph: "
                         "--layers layers of prologue + attention at S=2048, H=4, eager vs one "
                         "HIP-graph replay (launch overhead)")
    ap.add_argument("--blk", type=int, default=128, choices=list(range(16, 257, 16)),
                    help="sparse: query and key tile size (128: the 128x128 workload; 64: the SLA "
                         "block size default)")
    ap.add_argument("--topk", type=float, default=0.25,
                    help="sparse: fraction of key tiles kept per query tile by score, plus the diagonal "
                         "(0.25: the 128x128 workload; 0.35: the SLA node's default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-clock", action="store_true",
                    help="dense: skip the shader-clock measurement (one profiled layer after the timed steps)")
    ap.add_argument("--no-split-tail", action="store_true",
                    help="dense: run h3a_attn_fwd (never splits the last round of tiles) instead of "
                         "h3a_attn_fwd_ws")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the timed region, run one device copy of this many MiB "
                         "(reference kernel for scaling FETCH_SIZE/WRITE_SIZE counters)")
    return ap.parse_args()


def _timed(step, steps, warmup, n_launch, torch, stream):
    """Run warm-up, then exactly `steps` timed steps bracketed by synchronisation;
    HIP events on the launch stream around every launch give the per-kernel average."""
    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(n_launch)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s_ in range(steps):
        step(evs[s_])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = [a.elapsed_time(b) for st in evs for a, b in st]
    return wall, sum(kern_ms) / len(kern_ms)


def _calib_copy(args, torch, dev):
    if args.calib_copy_mib > 0:
        src = torch.empty(args.calib_copy_mib << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst


def _base(args, metric, value, unit, ms_per_step, config, higher=True):
    return {"metric": metric, "value": round(value, 2), "unit": unit, "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3),
            "higher_is_better": higher, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded device RNG, resident in HBM)", "config": config}


def run_dense(args, torch, h3attn, dev, heads=H):
    L = args.layers
    qs, ks, vs = [], [], []
    for layer in range(L):
        g = torch.Generator(device=dev).manual_seed(1000 + layer)
        qs.append(torch.randn(B, heads, S, D, generator=g, device=dev, dtype=torch.bfloat16))
        ks.append(torch.randn(B, heads, S, D, generator=g, device=dev, dtype=torch.bfloat16))
        vs.append(torch.randn(B, heads, S, D, generator=g, device=dev, dtype=torch.bfloat16).mul_(4))
    out = torch.empty(B, heads, S, D, device=dev, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)

    def step(events):
        for layer in range(L):
            if events is not None:
                events[layer][0].record(stream)
            h3attn.attn_fwd(qs[layer], ks[layer], vs[layer], out=out, split_tail=not args.no_split_tail)
            if events is not None:
                events[layer][1].record(stream)

    wall, avg_kernel_ms = _timed(step, args.steps, args.warmup, L, torch, stream)
    _calib_copy(args, torch, dev)
    fpl = flops_per_layer(h=heads)
    value = fpl * L * args.steps / wall / 1e12
    achieved = fpl / (avg_kernel_ms * 1e-3) / 1e12
    if heads == H:
        metric = "attn TFLOP/s & % bf16 MFMA peak at H=56,S=42120,D=128; ms per 50-layer step"
        workload = f"dense exact non-causal attention, {L} layers per step"
    else:
        metric = f"attn TFLOP/s & % bf16 MFMA peak at H={heads},S=42120,D=128 (one GPU's head share)"
        workload = f"dense exact non-causal attention, H={heads} share, {L} layers per step"
    res = _base(args, metric, value, "TFLOP/s", wall * 1e3 / args.steps,
                {"workload": workload, "B": B, "H": heads, "S": S, "D": D, "layers": L,
                 "segments": "text 512 + cond 256 + audio 2048 + video 39304"})
    res["data"] = "synthetic (seeded device RNG, fresh q/k/v per layer, resident in HBM)"
    traffic, traffic_src = measured_traffic() if heads == H else (None, "counters taken at H=56 only")
    ghz, clock_note = measure_clock(torch, h3attn, dev, heads) if not args.no_clock else (None, "skipped")
    roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic, "traffic_source": traffic_src,
            "kernel": "attn_fwd_pingpong_kernel (+ split_combine_kernel for the split tail)",
            "flop_per_launch": fpl, "avg_launch_ms": round(avg_kernel_ms, 3),
            "clock_ghz_measured": None if ghz is None else round(ghz, 3), "clock_note": clock_note}
    if ghz:
        peak_at_clock = FLOP_PER_CLK * ghz * 1e9 / 1e12
        roof["peak_at_measured_clock"] = round(peak_at_clock, 1)
        roof["frac_at_measured_clock"] = round(achieved / peak_at_clock, 4)
    res.update({
        "pct_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "ms_per_layer": round(avg_kernel_ms, 3),
        "roofline": roof,
    })
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(heads=heads)
        res["cpu_baseline"]["config1_sdpa_cpu"] = cpu_config1(torch)
    return res


def run_sparse(args, torch, h3attn, dev):
    """Block-sparse (h3_sla path): blk x blk tiles (128 by default: 330 per head at S=42120),
    top floor(topk*nk) key tiles per query tile from mean-pooled scores plus the diagonal
    (82 of 330 at 128 and topk 0.25); FLOPs counted exactly from the map."""
    from h3attn import ops, sla
    L, blk, topk = args.layers, args.blk, args.topk
    if not 0.0 < topk <= 1.0:
        raise SystemExit(f"--topk {topk}: must lie in (0, 1]")
    nk = (S + blk - 1) // blk
    tiles = blk not in ops.NATIVE_BLOCKS
    items = []
    map_ms = []
    for layer in range(L):
        g = torch.Generator(device=dev).manual_seed(2000 + layer)
        q = torch.randn(B, H, S, D, generator=g, device=dev, dtype=torch.bfloat16)
        k = torch.randn(B, H, S, D, generator=g, device=dev, dtype=torch.bfloat16)
        v = torch.randn(B, H, S, D, generator=g, device=dev, dtype=torch.bfloat16).mul_(4)
        a, b_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        bmap, lut, cnt = sla.get_block_map(q, k, topk, blk, blk, force_diag=True, smooth_k=False)
        if tiles:  # block sizes outside the native kernels': 32-key columns with sub-block masks
            lut, cnt = ops.block_map_to_tile_lut(bmap, blk, blk, S, S)
        b_.record()
        torch.cuda.synchronize()
        map_ms.append(a.elapsed_time(b_))
        nq = bmap.shape[2]
        valid = torch.full((nq,), blk, dtype=torch.float64, device=dev)
        valid[-1] = S - (nq - 1) * blk
        pairs = (bmap.double() * valid.view(1, 1, nq, 1) * valid.view(1, 1, 1, nq)).sum().item()
        items.append((q, k, v, lut, cnt, 4.0 * D * pairs))
    out = torch.empty(B, H, S, D, device=dev, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)

    def step(events):
        for i, (q, k, v, lut, cnt, _) in enumerate(items):
            if events is not None:
                events[i][0].record(stream)
            if tiles:
                ops.attn_fwd_blocksparse_tiles(q, k, v, lut, cnt, out=out)
            else:
                h3attn.attn_fwd_blocksparse(q, k, v, lut, cnt, blk, blk, out=out)
            if events is not None:
                events[i][1].record(stream)

    wall, avg_kernel_ms = _timed(step, args.steps, args.warmup, L, torch, stream)
    _calib_copy(args, torch, dev)
    ghz, clock_note = measure_clock_sparse(items[0], blk, tiles) if not args.no_clock else (None, "skipped")
    flops = sum(it[5] for it in items) / L
    value = flops * L * args.steps / wall / 1e12
    achieved = flops / (avg_kernel_ms * 1e-3) / 1e12
    res = _base(args, "block-sparse attn TFLOP/s (exact kept-tile FLOPs) at H=56,S=42120,D=128, "
                      f"{blk}x{blk} tiles, top-{round(100 * topk)}%+diagonal", value, "TFLOP/s",
                wall * 1e3 / args.steps,
                {"workload": f"block-sparse attention, {L} layers per step", "B": B, "H": H, "S": S,
                 "D": D, "blk_q": blk, "blk_k": blk,
                 "keep": f"{sla.keep_count(topk, nk)} of {nk} key tiles + diagonal"})
    if topk == 0.25:  # the counter summaries were measured at this keep ratio
        traffic, traffic_src = measured_traffic(TILES_TRAFFIC_SUMMARY if tiles else SPARSE_TRAFFIC_SUMMARY,
                                                f"sparse{blk}")
    else:
        traffic, traffic_src = None, "counters measured at --topk 0.25 only"
    res.update({
        "ms_per_layer": round(avg_kernel_ms, 3),
        "kept_fraction": round(flops / flops_per_layer(), 4),
        "dense_equivalent_tflops": round(flops_per_layer() / (avg_kernel_ms * 1e-3) / 1e12, 1),
        "block_map_ms": round(sum(map_ms[1:]) / max(1, len(map_ms) - 1), 3),
        "block_map_pooled_in_prologue": fused_pool_cost(torch, h3attn, dev, blk, topk),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": ("attn_fwd_pingpong_kernel<SwzLayout,2,sparse,key-split,tile-mask> (pairs of "
                                "64-row query blocks over 32-key columns with 16x16 sub-block masks)" if tiles
                                else "attn_fwd_pingpong_kernel<SwzLayout,2,sparse> (pairs of 128-row query blocks; "
                                "+ split_combine_kernel for the split tail)" if blk % 128 == 0
                                else "attn_fwd_pingpong_kernel<SwzLayout,2,sparse,key-split> (pairs of 64-row "
                                     "query blocks)"), "flop_per_launch": flops,
                     "avg_launch_ms": round(avg_kernel_ms, 3),
                     "clock_ghz_measured": None if ghz is None else round(ghz, 3), "clock_note": clock_note},
    })
    if ghz:
        peak_at_clock = FLOP_PER_CLK * ghz * 1e9 / 1e12
        res["roofline"]["peak_at_measured_clock"] = round(peak_at_clock, 1)
        res["roofline"]["frac_at_measured_clock"] = round(achieved / peak_at_clock, 4)
    return res


def fused_pool_cost(torch, h3attn, dev, blk, topk=0.25, reps=10):
    """Block-map cost when the prologue pools (h3a_qk_rmsnorm_rope_pool), at H=56, S=42120: median
    ms of the prologue alone, of the prologue with pooling at `blk`, and of the selection from
    those means (top 25 % + diagonal), each over `reps` launches on fused [S,3HD] views."""
    from h3attn import ops, sla
    qkv, qw, kw = _prologue_inputs(torch, dev, S, H, 11)
    rope = h3attn.rope_freqs(S, 128, device=dev)
    q = qkv[:, :H * D].view(1, S, H, D)
    k = qkv[:, H * D:2 * H * D].view(1, S, H, D)
    nk = (S + blk - 1) // blk

    def med(fn):
        ms = []
        for _ in range(reps + 1):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            out = fn()
            b.record()
            torch.cuda.synchronize()
            ms.append(a.elapsed_time(b))
        return sorted(ms[1:])[len(ms[1:]) // 2], out

    plain, _ = med(lambda: ops.qk_rmsnorm_rope_(q, k, rope, qw, kw, rot_dim=128))
    pooled, (pq, pk) = med(lambda: ops.qk_rmsnorm_rope_(q, k, rope, qw, kw, rot_dim=128, pool_blk=blk))
    select, _ = med(lambda: ops.block_select(pq, pk, sla.keep_count(topk, nk), blk, blk, force_diag=True,
                                             want_map=blk not in ops.NATIVE_BLOCKS))
    del qkv
    return {"prologue_ms": round(plain, 3), "prologue_pool_ms": round(pooled, 3),
            "block_select_ms": round(select, 3),
            "block_map_fused_ms": round(pooled - plain + select, 3),
            "note": "prologue (qk-RMSNorm+RoPE) at H=56, S=42120 alone and with the block pooling fused in; "
                    "block_map_fused_ms = the pooling's extra prologue time + the selection"}


def _prologue_inputs(torch, dev, s_len, heads, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    qkv = torch.randn(s_len, 3 * heads * D, generator=g, device=dev, dtype=torch.float32)
    spread = torch.empty(s_len, 1, device=dev).uniform_(0.5, 4.0, generator=g)
    qkv[:, :2 * heads * D] *= spread
    qkv = qkv.to(torch.bfloat16)
    qw = (1 + 0.05 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kw = (1 + 0.05 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    return qkv, qw, kw


def prologue_bytes(s_len=8192, heads=H, rot=128):
    return 4.0 * s_len * heads * D * 2 + s_len * (rot // 2) * 16 + 2 * D * 2


def run_prologue(args, torch, h3attn, dev):
    """qk-RMSNorm+RoPE in place on [S, 3*H*D] fused QKV views, S=8192, H=56, rot 128."""
    s_len, rot = 8192, 128
    qkv, qw, kw = _prologue_inputs(torch, dev, s_len, H, 7)
    rope = h3attn.rope_freqs(s_len, rot, device=dev)
    q = qkv[:, :H * D].view(1, s_len, H, D)
    k = qkv[:, H * D:2 * H * D].view(1, s_len, H, D)
    stream = torch.cuda.current_stream(dev)
    n = 20
    # One call takes about as long on the host (Python + ctypes) as the kernel
    # on the GPU.  A short spin on the stream first lets the host queue the
    # whole step, so the launches run back to back and the per-launch events
    # time the kernel rather than host gaps.
    prime_cycles = 20_000_000

    def step(events):
        torch.cuda._sleep(prime_cycles)
        for i in range(n):
            if events is not None:
                events[i][0].record(stream)
            h3attn.rms_rope_split_half_(q, k, rope, qw, kw, epsilon=1e-6, rot_dim=rot)
            if events is not None:
                events[i][1].record(stream)

    evs_all = []

    def step_rec(events):
        step(events)
        if events is not None:
            evs_all.append(events)

    _, avg_kernel_ms = _timed(step_rec, args.steps, args.warmup, n, torch, stream)
    # Whole-job GPU time: first launch start to last launch end of each step.
    span_ms = sum(ev[0][0].elapsed_time(ev[-1][1]) for ev in evs_all)
    _calib_copy(args, torch, dev)
    nbytes = prologue_bytes(s_len, H, rot)
    gbs = nbytes / (avg_kernel_ms * 1e-3) / 1e9
    traffic, traffic_src = measured_traffic(PROLOGUE_TRAFFIC_SUMMARY, "prologue")
    res = _base(args, "qk-RMSNorm+RoPE prologue GB/s (algorithmic bytes) at S=8192,H=56,D=128",
                nbytes * n * args.steps / (span_ms * 1e-3) / 1e9, "GB/s", span_ms / args.steps,
                {"workload": f"in-place qk-RMSNorm + split-half RoPE on fused-QKV views, {n} calls per step "
                             "(GPU span of the step's launches, queued behind a stream spin)",
                 "S": s_len, "H": H, "D": D, "rot_dim": rot, "qkv_row_stride": 3 * H * D})
    res.update({
        "us_per_call": round(avg_kernel_ms * 1e3, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(gbs / 8000.0, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": "qk_rmsnorm_rope_kernel", "bytes_per_launch": nbytes,
                     "avg_launch_ms": round(avg_kernel_ms, 4)},
    })
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_prologue_baseline(torch, s_len, rot)
    return res


def run_fused(args, torch, h3attn, dev):
    """One H3 block's attention on the fused QKV layout: prologue in place, then attention
    reading strided views and writing [S, H*D], S=8192, H=56, rot 128."""
    s_len, rot = 8192, 128
    qkv, qw, kw = _prologue_inputs(torch, dev, s_len, H, 9)
    rope = h3attn.rope_freqs(s_len, rot, device=dev)
    base = qkv.clone()
    q = qkv[:, :H * D].view(1, s_len, H, D)
    k = qkv[:, H * D:2 * H * D].view(1, s_len, H, D)
    v = qkv[:, 2 * H * D:].view(1, s_len, H, D)
    out = torch.empty(1, s_len, H, D, device=dev, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream(dev)
    n = 10

    def step(events):
        for i in range(n):
            qkv.copy_(base)  # fresh pre-norm inputs each call (outside the timed events)
            if events is not None:
                events[i][0].record(stream)
            h3attn.rms_rope_split_half_(q, k, rope, qw, kw, epsilon=1e-6, rot_dim=rot)
            h3attn.attn_fwd(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                            out=out.transpose(1, 2))
            if events is not None:
                events[i][1].record(stream)

    wall, avg_ms = _timed(step, args.steps, args.warmup, n, torch, stream)
    fl = flops_per_layer(h=H, s=s_len)
    tf = fl / (avg_ms * 1e-3) / 1e12
    res = _base(args, "fused block attention (prologue + attention) TFLOP/s at S=8192,H=56,D=128",
                tf, "TFLOP/s", wall * 1e3 / args.steps,
                {"workload": f"prologue + attention on fused [S,3HD] views, O as [S,HD], {n} calls per step",
                 "S": s_len, "H": H, "D": D, "rot_dim": rot})
    res.update({"ms_per_block": round(avg_ms, 3),
                "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None,
                             "kernel": "qk_rmsnorm_rope_kernel + attn_fwd_pingpong_kernel",
                             "flop_per_launch": fl, "avg_launch_ms": round(avg_ms, 3)}})
    return res


def run_graph(args, torch, h3attn, dev):
    """Launch overhead of a layer sequence: `--layers` layers of in-place prologue + dense
    attention on the fused QKV layout at S=2048, H=4 (per-layer GPU work of tens of
    microseconds), run eagerly from Python and as one HIP-graph replay (h3attn.graphs)."""
    from h3attn import graphs

    s_len, heads, rot = 2048, 4, 128
    rope = h3attn.rope_freqs(s_len, rot, device=dev)
    layers = []
    for i in range(args.layers):
        qkv, qw, kw = _prologue_inputs(torch, dev, s_len, heads, 100 + i)
        layers.append({"qkv": qkv, "rope": rope, "qw": qw, "kw": kw})
    # The prologue renormalises its inputs in place every pass; RMSNorm keeps them bounded,
    # so repeated passes are valid timing input.
    seq = graphs.LayerSequence(layers, heads=heads)

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / args.steps

    eager_s = timed(seq.run)
    seq.capture(warmup=1)
    graph_s = timed(seq.replay)
    fl = flops_per_layer(h=heads, s=s_len) * args.layers
    res = _base(args, f"HIP-graph replay of {args.layers} layers (prologue + attention) at S=2048,H=4: "
                      "attention TFLOP/s", fl / graph_s / 1e12, "TFLOP/s", graph_s * 1e3,
                {"workload": f"{args.layers} x (in-place prologue + dense attention) on fused [S,3HD] "
                             "views, one HIP graph", "S": s_len, "H": heads, "D": D, "rot_dim": rot})
    res.update({"ms_per_step_eager": round(eager_s * 1e3, 3), "ms_per_step_graph": round(graph_s * 1e3, 3),
                "us_per_layer_eager": round(eager_s * 1e6 / args.layers, 1),
                "us_per_layer_graph": round(graph_s * 1e6 / args.layers, 1),
                "graph_speedup": round(eager_s / graph_s, 2)})
    return res


def cpu_prologue_baseline(torch, s_len, rot):
    """A torch fp32 CPU restatement of the prologue (the reference has no CPU path)."""
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, s_len, H, D, generator=g).to(torch.bfloat16)
    w = torch.ones(D)
    half = rot // 2
    ang = torch.arange(s_len, dtype=torch.float32)[:, None] * (10000.0 ** (-2.0 * torch.arange(half) / rot))
    c, s_ = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]

    def once():
        y = x.float()
        y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + 1e-6) * w
        a, b_ = y[..., :half], y[..., half:rot]
        return torch.cat([a * c - b_ * s_, a * s_ + b_ * c, y[..., rot:]], -1).to(torch.bfloat16)

    once()
    t0 = time.perf_counter()
    reps = 3
    for _ in range(reps):
        once()
    dt = (time.perf_counter() - t0) / reps
    return {"value": round(prologue_bytes(s_len, H, rot) / dt / 1e9, 2), "unit": "GB/s", "cores": threads,
            "kind": "port", "sample": f"torch fp32 CPU restatement, full S={s_len} H={H}, {reps} reps, "
                                      f"{dt * 1e3:.0f} ms/call; CPU: {cpu_model()}"}


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported "
              "(the attention path runs on one GPU; it shards by heads across GPUs)", file=sys.stderr)
        sys.exit(2)

    import torch
    import h3attn

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload == "dense":
        res = run_dense(args, torch, h3attn, dev)
    elif args.workload == "h14":
        res = run_dense(args, torch, h3attn, dev, heads=14)
    elif args.workload == "sparse":
        res = run_sparse(args, torch, h3attn, dev)
    elif args.workload == "prologue":
        res = run_prologue(args, torch, h3attn, dev)
    elif args.workload == "graph":
        res = run_graph(args, torch, h3attn, dev)
    else:
        res = run_fused(args, torch, h3attn, dev)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
