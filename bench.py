#!/usr/bin/env python3
"""Q8 quantized-linear decode benchmark on one MI355X (gfx950).

Workload: the Qwen-27B-class Q8 decode projection set at
hidden 5120 -- fused QKV [7168 x 5120], o_proj [5120 x 6144], gate+up
[34816 x 5120], down [5120 x 17408] -- with weights N(0, 0.02) packed to
q8_g32_fp16 on the device and fp16 N(0, 1) activations, run at token counts
M in {1, 4, 8, 16}. A step is one pass of the 16 (projection, M) launches.
The timed region runs, for every (projection, M), K launches back to back
between one pair of HIP events on the launch stream, rotating independent
weight copies (at least 600 MB per projection) so that no launch is served
from the 256 MB Infinity Cache.

Printed JSON (one line): `value` is the whole-job algorithmic throughput in
GB/s (weights N*Kp*(1+2/32) + activations M*K*2 + outputs M*N*2, per launch)
over the timed region's wall clock; `roofline` divides the same bytes by the
summed event-measured kernel time; `per_launch` gives each kernel's average
launch duration; `cpu_baseline` times the reference's CPU path (torch FP32
GEMM over materialised weights) on a bounded sample of the same workload.
"""

import argparse
import json
import os
import platform
import sys
import time

import torch

PROJECTIONS = (("qkv", 7168, 5120), ("o_proj", 5120, 6144), ("gate_up", 34816, 5120), ("down", 5120, 17408))
TOKENS = (1, 4, 8, 16)
HBM_PEAK_GBS = 8000.0


def launch_bytes(m, n, k):
    padded = (k + 127) // 128 * 128
    return n * padded + n * (padded // 32) * 2 + m * k * 2 + m * n * 2


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--route", default="auto", choices=("auto", "exact", "mfma"))
    p.add_argument("--copy-mb", type=float, default=600.0, help="minimum rotated weight bytes per projection")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    return p.parse_args()


def build_copies(backend, device, copy_mb):
    """Per projection, enough independent packed copies to exceed `copy_mb` MB."""
    copies = []
    for i, (name, n, k) in enumerate(PROJECTIONS):
        count = max(2, -(-int(copy_mb * 1e6) // launch_bytes(0, n, k)))
        residents = []
        for c in range(count):
            gen = torch.Generator(device=device).manual_seed(1000 * c + i)
            w = torch.randn(n, k, generator=gen, device=device, dtype=torch.float32) * 0.02
            packed = backend.quantize_q8(w)
            del w
            residents.append(backend.upload_linear(packed, dtype=torch.float16, device=device))
            del packed
        copies.append(residents)
    torch.cuda.synchronize(device)
    return copies


def cpu_baseline(copies, xs, seconds):
    """Reference CPU path on copy 0 of the weights; same M values and inputs."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle.cpu_path import CpuQuantizedLinear, cpu_threads, time_calls

    threads = cpu_threads()
    layers = []
    for residents, (_, n, k) in zip(copies, PROJECTIONS):
        resident = residents[0]
        codes, scales = (t.cpu() for t in resident.storage_tensors)
        layers.append((CpuQuantizedLinear(codes, scales, k), n, k))
    calls, step_bytes = [], 0
    for m in TOKENS:
        for layer, n, k in layers:
            calls.append(lambda layer=layer, x=xs[m][k].cpu(): layer.run(x))
            step_bytes += launch_bytes(m, n, k)
    reps, elapsed = time_calls(calls, seconds)
    return {
        "value": round(reps * step_bytes / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} repetitions of the full config-2 step (4 projections x M in {list(TOKENS)}), "
        f"torch {torch.__version__} CPU GEMM, FP32 weights materialised before timing, "
        f"{elapsed:.1f} s on {platform.processor() or platform.machine()}",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from venturi_amd import create_backend

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    backend = create_backend("hip")
    copies = build_copies(backend, device, args.copy_mb)
    gen = torch.Generator(device=device).manual_seed(7)
    xs = {m: {k: torch.randn(m, k, generator=gen, device=device).half() for k in {p[2] for p in PROJECTIONS}}
          for m in TOKENS}
    outs = {(m, n): torch.empty(m, n, dtype=torch.float16, device=device) for m in TOKENS for (_, n, _) in PROJECTIONS}
    launches = [(mi, pi) for mi in range(len(TOKENS)) for pi in range(len(PROJECTIONS))]
    plans = {(mi, pi): [r.prepare(tokens=TOKENS[mi], route=args.route) for r in copies[pi]] for mi, pi in launches}
    routes = sorted({p[0].route for p in plans.values()})
    step_bytes = sum(launch_bytes(TOKENS[mi], PROJECTIONS[pi][1], PROJECTIONS[pi][2]) for mi, pi in launches)
    stream = torch.cuda.current_stream(device)

    def run(mi, pi, reps, events=None):
        m, (_, n, k) = TOKENS[mi], PROJECTIONS[pi]
        rotation = plans[(mi, pi)]
        if events is not None:
            events[0].record(stream)
        for s in range(reps):
            rotation[s % len(rotation)].run(xs[m][k], out=outs[(m, n)])
        if events is not None:
            events[1].record(stream)

    for mi, pi in launches:
        run(mi, pi, args.warmup)
    torch.cuda.synchronize(device)

    events = {key: [torch.cuda.Event(enable_timing=True) for _ in range(2)] for key in launches}
    torch.cuda.synchronize(device)
    start = time.perf_counter()
    for mi, pi in launches:
        run(mi, pi, args.steps, events[(mi, pi)])
    torch.cuda.synchronize(device)
    wall = time.perf_counter() - start

    kernel_s = {key: e[0].elapsed_time(e[1]) / 1e3 for key, e in events.items()}
    total_bytes = args.steps * step_bytes
    detail = {}
    for mi, pi in launches:
        m, (name, n, k) = TOKENS[mi], PROJECTIONS[pi]
        avg = kernel_s[(mi, pi)] / args.steps
        detail[f"{name}_m{m}"] = {"us": round(avg * 1e6, 2), "GB/s": round(launch_bytes(m, n, k) / avg / 1e9, 1),
                                  "route": plans[(mi, pi)][0].route}
    achieved = total_bytes / sum(kernel_s.values()) / 1e9

    result = {
        "metric": "Q8 quantlinear decode GB/s (M<=16), config-2 projection set",
        "value": round(total_bytes / wall / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: weights N(0,0.02) packed to q8_g32_fp16 on device, activations N(0,1) fp16",
        "config": {
            "workload": "config2: Qwen-27B-class Q8 decode projection set, hidden 5120, M in {1,4,8,16}",
            "projections": {p[0]: [p[1], p[2]] for p in PROJECTIONS},
            "tokens": list(TOKENS),
            "weight_copies": {p[0]: len(c) for p, c in zip(PROJECTIONS, copies)},
            "routes": routes,
            "bytes_per_step": step_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
        },
        "per_launch": detail,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(copies, xs, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
