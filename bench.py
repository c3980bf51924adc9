"""Benchmark of the group-64 packed-integer linear path on one MI355X.

Workload: the linears of a Llama-2-7B-shaped
decoder layer (q/k/v/o 4096x4096, gate/up 4096->11008, down 11008->4096),
W4A8 group-64, synthetic activations N(0,1) with 1 % outlier channels x10
and synthetic packed W4 codes + per-channel scales, over `--layers` layers
of distinct weights (1.2 GB at the default 12 layers, well above the 256 MB
Infinity Cache). One step = one pass over the stack at M=1 token: for every
linear the group-64 quantizer and the packed GEMM (actune_grouped_forward),
all captured in one hipGraph. Inputs are resident in HBM; `value` is the
packed-weight bytes streamed per second over the whole step.

Printed JSON line: the driver's contract fields plus
  roofline      the dominant kernel (small-M packed GEMM, gemm_smallm) timed
                with HIP events on its own stream over a GEMM-only graph of
                the same stack: algorithmic bytes / average launch duration
                vs 8 TB/s;
  cpu_baseline  the reference's dequantize-then-matmul path in torch-CPU
                (oracle/cpu_path.py) on a bounded sample (rank 0, N=1);
  detail        M=8 pass, per-shape us/launch, quantizer share.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBPS = 8000.0
SHAPES = [("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
          ("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008)]
METRIC = "µs per packed linear + achieved int8 TOPS / HBM GB/s vs roofline, per W/A config"


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--layers", type=int, default=12)
    p.add_argument("--W", type=int, default=4)
    p.add_argument("--A", type=int, default=8)
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a 1 GiB device copy (for PMC byte-counter calibration)")
    return p.parse_args()


def build_stack(torch, m, layers, W, A, seed=0):
    """Per layer and shape: packed weights, scales, input, scratch, output."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = "cuda"
    inputs = {}
    for _, n, k in SHAPES:
        if k not in inputs:
            x = torch.randn(m, k, generator=g, device=dev)
            ch = torch.randperm(k, generator=g, device=dev)[: k // 100]
            x[:, ch] *= 10
            inputs[k] = x.to(torch.bfloat16).contiguous()
    stack = []
    for _ in range(layers):
        for name, n, k in SHAPES:
            w = torch.randint(0, 256, (n, k * W // 8), generator=g, device=dev, dtype=torch.uint8)
            ws = torch.rand(n, generator=g, device=dev) * 0.01 + 0.005
            stack.append(dict(name=name, n=n, k=k, w=w, ws=ws, x=inputs[k],
                              a=torch.empty(m, k * A // 8, device=dev, dtype=torch.uint8),
                              s=torch.empty(m, k // 64, device=dev, dtype=torch.float32),
                              out=torch.empty(m, n, device=dev, dtype=torch.bfloat16)))
    return stack


def capture(torch, fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return graph


def time_graph(torch, graph, steps, warmup):
    """Milliseconds per replay, HIP events on the replay stream."""
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def gemm_bytes(n, k, m, W, A):
    """Algorithmic bytes of one GEMM launch: packed weights + weight scales +
    packed activations + activation scales + bf16 output."""
    return n * k * W // 8 + 4 * n + m * k * A // 8 + 4 * m * (k // 64) + 2 * m * n


def cpu_baseline(seconds, W, A):
    """Reference dequant-then-matmul (hoisted weight dequant) on one decoder
    layer's 7 linears at M=1, repeated for about `seconds`."""
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import cpu_path
    cores = min(16, os.cpu_count() or 1)
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    lo = -(1 << (W - 1))
    layer = []
    for _, n, k in SHAPES:
        codes = torch.randint(lo, -lo, (n, k), generator=g, dtype=torch.int8)
        scale = torch.rand(n, generator=g) * 0.01 + 0.005
        x = torch.randn(1, k, generator=g).to(torch.bfloat16)
        layer.append((x, cpu_path.dequantize_weight(codes, scale), n * k * W // 8))
    for x, wd, _ in layer:  # warm-up
        cpu_path.linear(x, A, wd)
    passes, nbytes, t0 = 0, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for x, wd, b in layer:
            cpu_path.linear(x, A, wd)
            nbytes += b
        passes += 1
    dt = time.perf_counter() - t0
    return dict(value=round(nbytes / dt / 1e9, 3), unit="GB/s (packed weight bytes)", cores=cores,
                kind="port",
                sample=f"{passes} passes over one Llama-2-7B layer's 7 linears at M=1, W{W}A{A}, "
                       f"torch-CPU fp32 dequant-then-matmul with hoisted weight dequant, "
                       f"{dt:.1f} s, {dt / passes / 7 * 1e6:.0f} us/linear")


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    import torch
    from actune_amd import _native
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps(dict(copy_bytes=1 << 30, launches=5)))
        return 0

    W, A = args.W, args.A
    results = {}
    for m in (1, 8):
        stack = build_stack(torch, m, args.layers, W, A)
        cfg = _native.default_config(m, 4096, 4096, W, A)

        def forward_pass():
            for e in stack:
                _native.grouped_forward(e["x"], e["w"], e["ws"], None, W, A, config=cfg, out=e["out"],
                                        packed=e["a"], scales=e["s"])

        def quant_pass():
            for e in stack:
                _native.quantize_groups(e["x"], A, packed=e["a"], scales=e["s"])

        def gemm_pass():
            for e in stack:
                _native.grouped_linear(e["a"], e["s"], e["w"], e["ws"], None, e["x"], W, A, cfg, out=e["out"])

        full = capture(torch, forward_pass)
        quant = capture(torch, quant_pass)
        gemm = capture(torch, gemm_pass)
        torch.cuda.synchronize()
        ms_full = time_graph(torch, full, args.steps, args.warmup)
        ms_gemm = time_graph(torch, gemm, args.steps, args.warmup)
        ms_quant = time_graph(torch, quant, args.steps, args.warmup)
        per_shape = {}
        for name, n, k in (SHAPES[0], SHAPES[4], SHAPES[6]):
            subset = [e for e in stack if e["name"] == name]

            def one_shape(subset=subset):
                for e in subset:
                    _native.grouped_linear(e["a"], e["s"], e["w"], e["ws"], None, e["x"], W, A, cfg, out=e["out"])

            gph = capture(torch, one_shape)
            us = time_graph(torch, gph, args.steps, args.warmup) * 1e3 / len(subset)
            per_shape[f"{n}x{k}"] = dict(us_per_launch=round(us, 3),
                                         weight_GBps=round(n * k * W / 8 / us / 1e3, 1))
            del gph
        wbytes = sum(e["n"] * e["k"] * W // 8 for e in stack)
        abytes = sum(gemm_bytes(e["n"], e["k"], m, W, A) for e in stack)
        ops = sum(2 * m * e["n"] * e["k"] for e in stack)
        results[m] = dict(ms_full=ms_full, ms_gemm=ms_gemm, ms_quant=ms_quant, wbytes=wbytes, abytes=abytes,
                          ops=ops, launches=len(stack), per_shape=per_shape, config=cfg)
        del full, quant, gemm, stack
        torch.cuda.synchronize()

    r1 = results[1]
    value = r1["wbytes"] / (r1["ms_full"] * 1e-3) / 1e9
    gemm_us = r1["ms_gemm"] * 1e3 / r1["launches"]
    achieved = r1["abytes"] / (r1["ms_gemm"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s (packed weight bytes per second, whole step)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r1["ms_full"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random packed W4 codes + scales; N(0,1) activations with 1% outlier channels x10)",
        "config": {"workload": "Llama-2-7B decoder linear stack (q,k,v,o,gate,up,down), batch 1, M=1 token",
                   "layers": args.layers, "W": W, "A": A, "group": 64, "M": 1,
                   "weight_bytes_per_step": r1["wbytes"], "launches_per_step": 2 * r1["launches"],
                   "gemm_config": r1["config"]},
        "us_per_linear": round(r1["ms_full"] * 1e3 / r1["launches"], 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "gemm_smallm (packed W4A8 GEMM, M=1)",
                     "avg_launch_us": round(gemm_us, 3)},
        "detail": {},
    }
    for m, r in results.items():
        line["detail"][f"M={m}"] = {
            "us_per_linear": round(r["ms_full"] * 1e3 / r["launches"], 3),
            "gemm_us_per_launch": round(r["ms_gemm"] * 1e3 / r["launches"], 3),
            "quant_us_per_launch": round(r["ms_quant"] * 1e3 / r["launches"], 3),
            "weight_GBps_whole_step": round(r["wbytes"] / (r["ms_full"] * 1e-3) / 1e9, 1),
            "weight_GBps_gemm_only": round(r["wbytes"] / (r["ms_gemm"] * 1e-3) / 1e9, 1),
            "int8_TOPS_gemm_only": round(r["ops"] / (r["ms_gemm"] * 1e-3) / 1e12, 3),
            "per_shape_gemm": r["per_shape"],
        }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds, W, A)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
