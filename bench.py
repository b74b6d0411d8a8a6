#!/usr/bin/env python3
"""Q8 quantized-linear decode benchmark on one MI355X (gfx950).

Workload (config 2): the Qwen-27B-class Q8 decode projection set at
hidden 5120 -- fused QKV [7168 x 5120], o_proj [5120 x 6144], gate+up
[34816 x 5120], down [5120 x 17408] -- with weights N(0, 0.02) packed to
q8_g32_fp16 on the device and fp16 N(0, 1) activations, run at token counts
M in {1, 4, 8, 16}. A step is one pass of the 16 (projection, M) launches.
For every (projection, M), K launches rotating independent weight copies (at
least 600 MB per projection, so that no launch is served from the 256 MB
Infinity Cache) are captured once in a HIP graph; the whole job (the 16
groups in turn) is also captured as one graph, whose replay is the timed
region of `value`, as a decode step runs in production; the 16 group graphs
are then replayed back to back, each between one pair of HIP events on the
launch stream, for the per-launch durations (every graph's output is checked
against an eager launch).

The line is compact by default: per-launch records are arrays over the token
counts `M` for each projection (`us`, and `GB/s` for the headline launches and
the exact route), agreement records keep their summary (and a max-ulp array per
launch); `--full` prints every record as its own object.

Printed JSON (one line): `value` is the whole-job algorithmic throughput in
GB/s (weights N*Kp*(1+2/32) + activations M*K*2 + outputs M*N*2, per launch)
over the timed region's wall clock; `roofline` is the dominant kernel's
algorithmic bytes over its own event-measured time, against the 8 TB/s HBM
peak; `per_launch` gives each launch's average duration; `parity` compares
every timed launch's output with the library's canonical-order route
(venturi_q8_head_run, byte-identical to the reference's kernel order: raw
max-abs, largest difference in fp16 ulps, outputs that differ, outputs more
than 2e-3 off, rel-L2); `exact_route` times that canonical route on the same
job; `cpu_baseline` times the reference's CPU path (torch FP32 GEMM over
materialised weights) on a bounded sample of the same workload. Further
sections of the same line carry their own roofline objects: `config1`
(config 1, 4096 x 4096 at one token, rotated copies), `vocab_head`
(the 248 320 x 5120 Q8 head held once in the tiled layout), `q4_decode`
(the metric's Q4 leg), `q56_decode`, `codecs`, `a8_decode` (the A8 path at
1 and 8 tokens, one and two passes), `prefill_a8` (config 3),
`prefill_a16` (W8A16 / W4A16 at M = 2048), `moe_w4a16` (config 4) and
`model_decode` (config 5).
"""

import argparse
import json
import os
import re
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
PROJECTIONS = (("qkv", 7168, 5120), ("o_proj", 5120, 6144), ("gate_up", 34816, 5120), ("down", 5120, 17408))
TOKENS = (1, 4, 8, 16)
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
FP16_PEAK_TFLOPS = 2500.0


def log(message):
    """Progress of the bench's own stages, on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def padded_k(k):
    return (k + 127) // 128 * 128


def launch_bytes(m, n, k):
    padded = padded_k(k)
    return n * padded + n * (padded // 32) * 2 + m * k * 2 + m * n * 2


def q4_launch_bytes(m, n, k):
    padded = padded_k(k)
    return n * padded // 2 + n * (padded // 64) * 2 + m * k * 2 + m * n * 2


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--route", default="auto", choices=("auto", "exact", "mfma"))
    p.add_argument("--copy-mb", type=float, default=600.0, help="minimum rotated weight bytes per projection")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    p.add_argument("--no-q4", action="store_true", help="skip the Q4 W4A16 and Q5/Q6 decode sections")
    p.add_argument("--no-prefill", action="store_true", help="skip the config-3 A8 and A16 prefill sections")
    p.add_argument("--no-moe", action="store_true", help="skip the config-4 routed-expert MoE section")
    p.add_argument("--no-model", action="store_true", help="skip the config-5 64-layer decode section")
    p.add_argument("--only", default=None,
                   help="comma-separated sections to run (config2,config1,head,q4,q56,codecs,a8dec,a8,a16,moe,model); "
                   "without config2 no headline metric is printed (for counter runs)")
    p.add_argument("--full", action="store_true",
                   help="print per-launch and per-projection records as one object each (the default line is compact)")
    p.add_argument("--eager", action="store_true",
                   help="time config-2 launches issued from Python instead of HIP-graph replays (for counter runs)")
    return p.parse_args()


# ---------------------------------------------------------------- helpers


def agreement(got, ref):
    """Raw agreement of fp16 outputs with reference-order fp16 outputs (device tensors).

    max_abs, max_ulp (largest difference in fp16 ulps of the reference value),
    flips (outputs that differ at all), over_2e-3, rel_l2, count.
    """
    g, r = got.double(), ref.double()
    diff = (g - r).abs()
    ulp = torch.exp2(torch.floor(torch.log2(r.abs().clamp_min(2.0**-14))) - 10)
    denom = float(torch.linalg.vector_norm(r))
    return {
        "max_abs": float(diff.max()),
        "max_ulp": float((diff / ulp).max()),
        "flips": int((diff > 0).sum()),
        "over_2e-3": int((diff > 2e-3).sum()),
        "rel_l2": float(torch.linalg.vector_norm(g - r)) / max(denom, 1e-30),
        "count": r.numel(),
    }


def merge_agreement(items):
    """Worst-case summary of several agreement records."""
    items = list(items)
    return {
        "max_abs": max(i["max_abs"] for i in items),
        "max_ulp": max(i["max_ulp"] for i in items),
        "flips": sum(i["flips"] for i in items),
        "over_2e-3": sum(i["over_2e-3"] for i in items),
        "max_rel_l2": max(i.get("rel_l2", i.get("max_rel_l2", 0.0)) for i in items),
        "count": sum(i["count"] for i in items),
    }


def compact(stats):
    return {k: (float(f"{v:.4g}") if isinstance(v, float) else v) for k, v in stats.items()}


_LAUNCH_KEY = re.compile(r"^(?P<proj>[a-z_]+?)_m(?P<m>\d+)(?P<suffix>_p\d+)?$")


def launch_table(detail):
    """Per-launch records keyed '<projection>_m<M>[_p<passes>]' as one array per field and projection.

    {'qkv_m1': {'us': 9.5, 'GB/s': 4120}, 'qkv_m4': ...} becomes
    {'M': [1, 4, ...], 'us': {'qkv': [9.5, ...]}, 'GB/s': {...}}; a string or
    boolean field that is the same in every record is kept once. Records of
    another shape are returned unchanged.
    """
    ms, numeric, uniform = [], {}, {}
    for key, rec in detail.items():
        hit = _LAUNCH_KEY.match(key)
        if hit is None or not isinstance(rec, dict):
            return detail
        m, name = int(hit["m"]), hit["proj"] + (hit["suffix"] or "")
        if m not in ms:
            ms.append(m)
        for field, v in rec.items():
            if isinstance(v, bool) or isinstance(v, str):
                uniform.setdefault(field, set()).add(v)
            elif isinstance(v, (int, float)):
                numeric.setdefault(field, {}).setdefault(name, {})[m] = v
    out = {"M": ms}
    for field, per in numeric.items():
        out[field] = {name: [vals.get(m) for m in ms] for name, vals in per.items()}
    for field, values in uniform.items():
        out[field] = values.pop() if len(values) == 1 else sorted(values, key=str)
    return out


# Sections of the printed line in order: the contract's fields first, then the
# sections least often read, so that a reader holding only the end of a long
# line still has the headline's per-launch table, parity and exact route.
_LINE_ORDER = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
               "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "timing", "all_kernels_GBps",
               "graph_equals_eager", "codecs", "config1", "q56_decode", "model_decode", "moe_w4a16", "prefill_a16",
               "prefill_a8", "a8_decode", "q4_decode", "vocab_head", "exact_route", "parity", "per_launch")


def shorten(result):
    """The printed line in compact form, so that the whole line stays a few KB.

    Per-launch records become arrays over M (`launch_table`); per-launch
    agreement records keep their max-ulp column (the section's summary holds
    the rest); per-projection agreement records are left to the summary;
    GB/s columns are kept for the headline's launches and the exact route and
    left out elsewhere (the section's own GB/s and roofline stay); stage
    fractions of peak are left out (their TFLOP/s / TOPS stay), and so are the
    prefill stages' TFLOP/s (the times stay), the library route's note and
    agreement record, the Q5/Q6 per-launch tables (their GB/s and roofline
    stay) and the section baselines' sample text (`--full` prints them all).
    """
    keep_rate = ("exact_route",)  # besides the headline's own per_launch

    def dropped(key, path):
        if key == "per_projection":
            return True
        if "stages" in path and (key.startswith("frac_") and key.endswith("_peak")
                                 or path[0] == "prefill_a16" and key == "TFLOP/s"):
            return True
        if path[-1:] == ("library_route",) and key in ("note", "parity"):
            return True
        if path[:1] == ("q56_decode",) and key == "per_launch":
            return True
        return path[1:] == ("cpu_baseline",) and key == "sample"

    def walk(node, path):
        if not isinstance(node, dict):
            return node
        out = {}
        for key, value in node.items():
            if dropped(key, path):
                continue
            if key == "per_launch" and isinstance(value, dict):
                sample = next(iter(value.values()), None)
                if isinstance(sample, dict) and "max_ulp" in sample:
                    table = launch_table({k: {"max_ulp": v["max_ulp"]} for k, v in value.items()})
                else:
                    table = launch_table({k: walk(v, path + (key,)) for k, v in value.items()})
                    if path and path[0] not in keep_rate and isinstance(table.get("GB/s"), dict) and "us" in table:
                        table.pop("GB/s")
                out[key] = table
            else:
                out[key] = walk(value, path + (key,))
        return out

    short = walk(result, ())
    ordered = {k: short[k] for k in _LINE_ORDER if k in short}
    ordered.update({k: v for k, v in short.items() if k not in ordered})
    return ordered


def event_time(fn, reps, warmup, stream):
    """Average seconds of fn() over `reps` back-to-back calls between two events on `stream`."""
    for _ in range(warmup):
        fn()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / 1e3 / reps


def graph_timing(groups, steps, warmup, device, eager=False):
    """Times launch groups through HIP graphs.

    ``groups`` maps a key to (run, verify): run(reps) issues `reps` launches
    (rotating weight copies); verify() re-runs the group's last launch eagerly
    and returns whether the group's output equals it. Each group's `steps`
    launches are captured in one graph, and the whole job (every group in
    turn) in another. Returns (seconds per group from events around its graph
    replay, wall seconds of one replay of the whole-job graph, graphs equal
    eager). With eager=True the launches are issued from Python between the
    events instead, and the wall time is that of the eager pass.
    """
    stream = torch.cuda.current_stream(device)
    for run, _ in groups.values():
        run(warmup)
    torch.cuda.synchronize(device)
    events = {key: [torch.cuda.Event(enable_timing=True) for _ in range(2)] for key in groups}
    if eager:
        start = time.perf_counter()
        for key, (run, _) in groups.items():
            events[key][0].record(stream)
            run(steps)
            events[key][1].record(stream)
        torch.cuda.synchronize(device)
        wall = time.perf_counter() - start
        return {k: e[0].elapsed_time(e[1]) / 1e3 for k, e in events.items()}, wall, None
    graphs = {}
    for key, (run, _) in groups.items():
        graphs[key] = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graphs[key]):
            run(steps)
    same = True
    for key, (_, verify) in groups.items():
        graphs[key].replay()
        torch.cuda.synchronize(device)
        same &= bool(verify())
    step_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(step_graph):
        for run, _ in groups.values():
            run(steps)
    step_graph.replay()
    torch.cuda.synchronize(device)
    for _, verify in groups.values():
        same &= bool(verify())
    start = time.perf_counter()
    step_graph.replay()
    torch.cuda.synchronize(device)
    wall = time.perf_counter() - start
    # One untimed replay of every group is queued first, so that the GPU is
    # busy while the timed replays are submitted: otherwise the first group's
    # events also hold the host's submission time after the synchronisation
    # (measured: +1.5 us per launch on the first group against its kernel trace).
    for key in groups:
        graphs[key].replay()
    for key in groups:
        events[key][0].record(stream)
        graphs[key].replay()
        events[key][1].record(stream)
    torch.cuda.synchronize(device)
    del graphs, step_graph
    return {k: e[0].elapsed_time(e[1]) / 1e3 for k, e in events.items()}, wall, same


def rotated_group(plans, x, out, steps):
    """(run, verify) of one launch group over rotated plans writing `out`."""

    def run(reps):
        for s in range(reps):
            plans[s % len(plans)].run(x, out=out)

    def verify():
        ref = torch.empty_like(out)
        plans[(steps - 1) % len(plans)].run(x, out=ref)
        torch.cuda.synchronize(out.device)
        return torch.equal(ref.view(torch.int16), out.view(torch.int16))

    return run, verify


def q8_copies(backend, device, shapes, copy_mb, seed):
    """Per (name, n, k), independent Q8 residents whose bytes exceed `copy_mb` MB."""
    copies = []
    for i, (name, n, k) in enumerate(shapes):
        count = max(2, -(-int(copy_mb * 1e6) // launch_bytes(0, n, k)))
        residents = []
        for c in range(count):
            gen = torch.Generator(device=device).manual_seed(seed + 1000 * c + i)
            w = torch.randn(n, k, generator=gen, device=device, dtype=torch.float32) * 0.02
            packed = backend.quantize_q8(w)
            del w
            residents.append(backend.upload_linear(packed, dtype=torch.float16, device=device))
            del packed
        copies.append(residents)
    torch.cuda.synchronize(device)
    return copies


def cpu_description(threads):
    from oracle.cpu_path import cpu_model

    return f"{threads} threads on {cpu_model()}, torch {torch.__version__}"


# ---------------------------------------------------------------- config 2


def decode_job(backend, device, copies, route, steps, warmup, eager):
    """The config-2 job on one route: per-launch seconds, wall seconds, graph check, outputs of copy 0."""
    gen = torch.Generator(device=device).manual_seed(7)
    xs = {m: {k: torch.randn(m, k, generator=gen, device=device).half() for k in {p[2] for p in PROJECTIONS}}
          for m in TOKENS}
    groups, outs, plans = {}, {}, {}
    for m in TOKENS:
        for pi, (name, n, k) in enumerate(PROJECTIONS):
            key = (m, name)
            plans[key] = [r.prepare(tokens=m, route=route) for r in copies[pi]]
            outs[key] = torch.empty(m, n, dtype=torch.float16, device=device)
            groups[key] = rotated_group(plans[key], xs[m][k], outs[key], steps)
    seconds, wall, same = graph_timing(groups, steps, warmup, device, eager)
    first = {}
    for (m, name), p in plans.items():
        k = dict((q[0], q[2]) for q in PROJECTIONS)[name]
        o = torch.empty_like(outs[(m, name)])
        p[0].run(xs[m][k], out=o)
        first[(m, name)] = o
    torch.cuda.synchronize(device)
    routes = {key: p[0].route for key, p in plans.items()}
    return seconds, wall, same, first, routes


def config2(backend, device, args):
    log("packing config-2 weight copies")
    copies = q8_copies(backend, device, PROJECTIONS, args.copy_mb, 0)
    step_bytes = sum(launch_bytes(m, n, k) for m in TOKENS for _, n, k in PROJECTIONS)
    log("config-2 decode: warm-up, graph capture and timed region")
    seconds, wall, same, outputs, routes = decode_job(backend, device, copies, args.route, args.steps, args.warmup,
                                                      args.eager)
    log("config-2 decode on the canonical-order route (timing and parity reference)")
    ex_seconds, ex_wall, ex_same, ex_outputs, _ = decode_job(backend, device, copies, "exact", args.steps,
                                                             max(1, args.warmup // 2), args.eager)
    total_bytes = args.steps * step_bytes
    detail, ex_detail, parity = {}, {}, {}
    by_route = {}
    for m in TOKENS:
        for name, n, k in PROJECTIONS:
            key, label = (m, name), f"{name}_m{m}"
            avg = seconds[key] / args.steps
            b = launch_bytes(m, n, k)
            detail[label] = {"us": round(avg * 1e6, 2), "GB/s": round(b / avg / 1e9, 1), "route": routes[key]}
            ex_avg = ex_seconds[key] / args.steps
            ex_detail[label] = {"us": round(ex_avg * 1e6, 2), "GB/s": round(b / ex_avg / 1e9, 1)}
            parity[label] = compact(agreement(outputs[key], ex_outputs[key]))
            bt = by_route.get(routes[key], (0, 0.0))
            by_route[routes[key]] = (bt[0] + args.steps * b, bt[1] + seconds[key])
    dominant = max(by_route, key=lambda r: by_route[r][1])
    achieved = by_route[dominant][0] / by_route[dominant][1] / 1e9
    kernels = {"venturi-q8-exact": "q8_exact (canonical order)",
               "venturi-q8-mfma": "q8_tiled_lds / q8_tiled_decode (fp16 MFMA)"}
    summary = merge_agreement(parity.values())
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
            "routes": sorted(set(routes.values())),
            "bytes_per_step": step_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kernels.get(dominant, dominant),
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(args.route),
        },
        "all_kernels_GBps": round(total_bytes / sum(seconds.values()) / 1e9, 1),
        "graph_equals_eager": same,
        "timing": ("eager launches" if args.eager else
                   "value: one HIP graph of the whole job (K steps x 16 launch groups), wall clock of its replay; "
                   "per_launch: one graph per group between HIP events"),
        "parity": {
            "against": "venturi_q8_head_run (canonical order, byte-identical to the reference's q8_head order; "
                       "checked against the oracle by tests/test_gpu_q8_exact.py)",
            "tolerance": "max-abs 2e-3 where |y| < 4; one fp16 ulp (3.9e-3) at |y| >= 4",
            "summary": compact(summary),
            "per_launch": parity,
        },
        "exact_route": {
            "kernel": "q8_exact (venturi_q8_head_run)",
            "GB/s": round(total_bytes / ex_wall / 1e9, 1),
            "kernels_GBps": round(total_bytes / sum(ex_seconds.values()) / 1e9, 1),
            "graph_equals_eager": ex_same,
            "per_launch": ex_detail,
        },
        "per_launch": detail,
    }
    return result, copies


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q8_decode_traffic.json")


def measured_traffic(route):
    """HBM bytes per launch of the config-2 step, from the committed counter runs.

    The figure comes from two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) over
    this bench's eager launches, each scaled by the same counter's reading for a
    copy of known size; the file records the commands and raw values. None when
    the file is absent or was measured on another route.
    """
    try:
        with open(TRAFFIC_FILE) as f:
            record = json.load(f)
    except (OSError, ValueError):
        return None
    if record.get("route") != route:
        return None
    return record.get("traffic_bytes_per_launch")


def cpu_baseline(copies, seconds):
    """Reference CPU path on copy 0 of the config-2 weights; same M values, seeded inputs."""
    from oracle.cpu_path import CpuQuantizedLinear, cpu_threads, time_calls

    threads = cpu_threads()
    layers = []
    for residents, (_, n, k) in zip(copies, PROJECTIONS):
        codes, scales = (t.cpu() for t in residents[0].storage_tensors[:2])
        layers.append((CpuQuantizedLinear(codes, scales, k), n, k))
    gen = torch.Generator().manual_seed(7)
    calls, step_bytes = [], 0
    for m in TOKENS:
        for layer, n, k in layers:
            x = torch.randn(m, k, generator=gen).half()
            calls.append(lambda layer=layer, x=x: layer.run(x))
            step_bytes += launch_bytes(m, n, k)
    reps, elapsed = time_calls(calls, seconds)
    return {
        "value": round(reps * step_bytes / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} repetitions of the full config-2 step (4 projections x M in {list(TOKENS)}), "
        f"FP32 weights materialised before timing, {elapsed:.1f} s; {cpu_description(threads)}",
    }


# ---------------------------------------------------------------- config 1


def config1(backend, device, steps, warmup, copy_mb):
    """Config 1: one q8_g32_fp16 [4096 x 4096] projection at one token.

    Weights N(0, 0.02) (copy 0 from seed 0), x fp16 N(0, 1) from seed 1. The
    17.8 MB matrix fits the 256 MB Infinity Cache, so each graph rotates
    >= `copy_mb` MB of independent copies (at least 2 x the copy count
    launches per graph); auto and canonical routes are timed alike and their
    outputs compared.
    """
    shape = (("w", 4096, 4096),)
    copies = q8_copies(backend, device, shape, copy_mb, 0)[0]
    x = torch.randn(1, 4096, generator=torch.Generator().manual_seed(1)).half().to(device)
    reps = max(steps, 2 * len(copies))
    b = launch_bytes(1, 4096, 4096)
    out, result = {}, {"workload": "config1: q8_g32_fp16 [4096 x 4096], M=1", "weight_copies": len(copies),
                       "launches_per_graph": reps, "bytes_per_launch": b}
    for route in ("auto", "exact"):
        plans = [r.prepare(tokens=1, route=route) for r in copies]
        out[route] = torch.empty(1, 4096, dtype=torch.float16, device=device)
        seconds, wall, same = graph_timing({route: rotated_group(plans, x, out[route], reps)}, reps, warmup, device)
        avg = seconds[route] / reps
        gbs = b / avg / 1e9
        result[route] = {"route": plans[0].route, "us": round(avg * 1e6, 3), "GB/s": round(gbs, 1),
                         "graph_equals_eager": same,
                         "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                      "frac": round(gbs / HBM_PEAK_GBS, 4)}}
        plans[0].run(x, out=out[route])
    torch.cuda.synchronize(device)
    result["parity_auto_vs_exact"] = compact(agreement(out["auto"], out["exact"]))
    return result


# ---------------------------------------------------------------- config 3


def prefill_a8(backend, device, steps, warmup, cpu_seconds):
    """Config 3: RMSNorm + 1-pass A8 at hidden 5120, int8 GEMMs at the config-2 shapes, M = 2048.

    x fp16 [2048, 5120] ~ N(0, 1) with 51 seeded channels (1%) scaled by 20;
    gamma ~ N(1, 0.1); eps 1e-6. QKV and gate+up consume the fused RMS+A8
    workspace; o_proj (K 6144) and down (K 17408) quantize seeded N(0, 1)
    activations with the plain A8 quantizer. Each stage runs `steps` times back
    to back between one pair of events; TOPS = 2*M*N*K / average time. The
    GEMMs run on the plan's auto route (matrix cores, natural group order);
    the reference-order route is timed beside it and its outputs are the
    parity reference.
    """
    from venturi_amd import prepare_q8_dp4a, prepare_rms_q8

    m = 2048
    gen = torch.Generator(device=device).manual_seed(3)
    x = torch.randn(m, 5120, generator=gen, device=device)
    outliers = torch.randperm(5120, generator=torch.Generator().manual_seed(3))[:51].to(device)
    x[:, outliers] *= 20
    x = x.half()
    gamma = (1 + 0.1 * torch.randn(5120, generator=gen, device=device)).float()
    norm = backend.upload_rmsnorm(gamma, dtype=torch.float16, device=device, epsilon=1e-6)
    rms_plan = prepare_rms_q8(norm, tokens=m, residual_compensation=False)
    stream = torch.cuda.current_stream(device)
    results, total_ops, total_s, exact_s, parity = {}, 0, 0.0, 0.0, {}
    ws_5120 = torch.empty(rms_plan.workspace_bytes, dtype=torch.uint8, device=device)
    results["rms_a8_k5120"] = {
        "us": round(event_time(lambda: rms_plan.run(x, workspace=ws_5120), steps, warmup, stream) * 1e6, 2),
        "bytes_per_token": 16000}
    cpu_layers = []
    for name, n, k in PROJECTIONS:
        packed = backend.quantize_q8(torch.randn(n, k, generator=gen, device=device) * 0.02)
        resident = backend.upload_linear(packed, dtype=torch.float16, device=device)
        if cpu_seconds > 0:
            cpu_layers.append((packed.codes.cpu(), packed.scales.cpu(), n, k))
        del packed
        plan = prepare_q8_dp4a(resident, tokens=m, residual_compensation=False)
        exact = prepare_q8_dp4a(resident, tokens=m, residual_compensation=False, route="exact")
        out = torch.empty(m, n, dtype=torch.float16, device=device)
        ref = torch.empty_like(out)
        if k == 5120:
            ws = ws_5120
        else:
            ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
            xa = torch.randn(m, k, generator=gen, device=device).half()
            results[f"a8_quantize_k{k}"] = {
                "us": round(event_time(lambda: plan.quantize(xa, workspace=ws), steps, warmup, stream) * 1e6, 2)}
        t = event_time(lambda: plan.project(out=out, workspace=ws), steps, warmup, stream)
        t_exact = event_time(lambda: exact.project(out=ref, workspace=ws), max(steps // 4, 2), 1, stream)
        torch.cuda.synchronize(device)
        parity[name] = compact(agreement(out, ref))
        ops = 2 * m * n * k
        total_ops += ops
        total_s += t
        exact_s += t_exact
        results[name] = {"us": round(t * 1e6, 1), "TOPS": round(ops / t / 1e12, 1),
                         "frac_int8_peak": round(ops / t / 1e12 / INT8_PEAK_TOPS, 4), "route": plan.route,
                         "exact_route_us": round(t_exact * 1e6, 1)}
        del resident, plan, exact, out, ref
    tops = total_ops / total_s / 1e12
    result = {
        "workload": "config3: RMSNorm+A8 (1 pass) -> int8 GEMMs at the config-2 shapes, M=2048",
        "gemm_TOPS": round(tops, 1),
        "exact_route_gemm_TOPS": round(total_ops / exact_s / 1e12, 1),
        "roofline": {"bound": "mfma", "kernel": "a8_gemm_fast", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS,
                     "unit": "TOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4)},
        "parity": {"against": "the reference-order route (venturi_q8_dp4a_run order, byte-identical to the oracle)",
                   "summary": compact(merge_agreement(parity.values())), "per_projection": parity},
        "stages": results,
    }
    if cpu_seconds > 0:
        from oracle.cpu_path import CpuA8Linear, cpu_threads, time_calls

        threads = cpu_threads()
        sample = 128
        cgen = torch.Generator().manual_seed(3)
        calls, ops = [], 0
        for codes, scales, n, k in cpu_layers:
            layer = CpuA8Linear(codes, scales, k, passes=1)
            xs = torch.randn(sample, k, generator=cgen).half()
            calls.append(lambda layer=layer, xs=xs: layer.run(xs))
            ops += 2 * sample * n * k
        reps, elapsed = time_calls(calls, cpu_seconds)
        result["cpu_baseline"] = {
            "value": round(reps * ops / elapsed / 1e12, 4), "unit": "TOP/s", "cores": threads, "kind": "oracle",
            "sample": f"{sample} of the 2048 tokens through the 4 projections ({reps} repetitions, {elapsed:.1f} s): "
            f"FP32 restatement of quantize_reference (1 pass) plus the FP32 matmul of the represented values "
            f"(the reference has no CPU int8 GEMM); {cpu_description(threads)}",
        }
    return result


def a8_decode(backend, device, steps, warmup, copy_mb, tokens_list=(1, 8)):
    """The A8 path at decode token counts (the reference's V100 benchmark case,
    benchmarks/v100-q8-dp4a/summary.md:101-110): the config-2 projection set,
    M in {1, 8}, one pass and two (the residual profile). Each launch quantizes
    the fp16 activations into the plan's workspace and runs the W8A8 projection
    (route auto: the int8 matrix-core decode kernel up to 32 tokens), rotating >=
    `copy_mb` MB of weight copies in one HIP graph per group, as the Q8 decode.
    Algorithmic bytes per launch = N*Kp*(1 + 2/32) weights + M*K*2 activations +
    2 * M*ceil(K/32)*36*passes workspace (written, read) + M*N*2 outputs.
    """
    from venturi_amd import prepare_q8_dp4a

    copies = q8_copies(backend, device, PROJECTIONS, copy_mb, 9000)
    gen = torch.Generator(device=device).manual_seed(23)
    xs = {m: {k: torch.randn(m, k, generator=gen, device=device).half() for k in {p[2] for p in PROJECTIONS}}
          for m in tokens_list}
    groups, nbytes, route = {}, {}, None
    for passes in (1, 2):
        for m in tokens_list:
            for pi, (name, n, k) in enumerate(PROJECTIONS):
                plans = [prepare_q8_dp4a(r, tokens=m, residual_compensation=passes == 2) for r in copies[pi]]
                route = plans[0].route
                ws = torch.empty(plans[0].workspace_bytes, dtype=torch.uint8, device=device)
                out = torch.empty(m, n, dtype=torch.float16, device=device)
                x = xs[m][k]

                def run(reps, plans=plans, x=x, out=out, ws=ws):
                    for r in range(reps):
                        plans[r % len(plans)].run(x, out=out, workspace=ws)

                def verify(plans=plans, x=x, out=out, ws=ws):
                    ref = torch.empty_like(out)
                    plans[(steps - 1) % len(plans)].run(x, out=ref, workspace=ws)
                    torch.cuda.synchronize(out.device)
                    return torch.equal(ref.view(torch.int16), out.view(torch.int16))

                key = (passes, m, name)
                groups[key] = (run, verify)
                nbytes[key] = launch_bytes(m, n, k) + 2 * m * -(-k // 32) * 36 * passes
    seconds, wall, same = graph_timing(groups, steps, warmup, device)
    detail, total = {}, 0
    for (passes, m, name), t in seconds.items():
        b = steps * nbytes[(passes, m, name)]
        total += b
        detail[f"{name}_m{m}_p{passes}"] = {"us": round(t / steps * 1e6, 2), "GB/s": round(b / t / 1e9, 1)}
    achieved = total / sum(seconds.values()) / 1e9
    return {
        "workload": "A8 decode: config-2 projection set, M in {1, 8}, 1 and 2 passes (quantize + W8A8 projection)",
        "route": route,
        "GB/s": round(total / wall / 1e9, 1),
        "roofline": {"bound": "hbm", "kernel": "a8 quantize + " + (
                         "int8 matrix-core W8A8 decode projection (a8_tiled_lds / a8_tiled_decode)" if route == "venturi-q8-a8-mfma"
                         else "reference-order W8A8 projection"),
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4)},
        "graph_equals_eager": same,
        "per_launch": detail,
    }


# ---------------------------------------------------------------- A16 prefill


def prefill_a16(backend, device, steps, warmup):
    """fp16-activation prefill GEMMs at the config-2 shapes, M = 2048 (the metric's
    "fp16 TOPS (M >= 256)" leg): W8A16 (q8_g32, venturi_q8_prefill_run) and W4A16
    (q4_g64), both on their plans' auto route, which at 2048 tokens is the dense
    one: W4A16 through venturi_row_dense_run (fp16 shadow chunks + hipBLASLt, the
    reference's ChunkedDense form), W8A16 through venturi_q8_dense_run (exact
    two-term fp16 weights over a doubled K). TFLOP/s counts 2*M*N*K either way;
    the hand-written matrix-core kernel on the same weights is timed beside it
    as `fused_mfma_us`, and `roofline` is that kernel's (the library route's
    figure is `library_route`).

    Weights N(0, 0.02) packed on the device; x fp16 N(0, 1). Each GEMM runs
    `steps` times back to back between one pair of events; TFLOP/s =
    2*M*N*K / average time, against the 2.5 PFLOP/s dense fp16 peak. Parity:
    W8A16 against the canonical-order route (venturi_q8_head_run); W4A16
    against the reference's own W4A16 path on this GPU (fp16(q*s) weights
    decoded by venturi_row_dequant_rows, then torch's fp16 linear with fp32
    accumulation, as the reference's dequant-then-F.linear path does). `parity`
    is the hand-written kernel's output; the library route's agreement is
    `library_route.parity` (for W4A16 that compares hipBLASLt with torch's
    linear, itself hipBLASLt on this GPU).
    """
    m = 2048
    gen = torch.Generator(device=device).manual_seed(11)
    stream = torch.cuda.current_stream(device)
    sections = {}
    for codec, quantize in (("w8a16", backend.quantize_q8), ("w4a16", backend.quantize_q4)):
        stages, total_flops, total_s, fused_s, route, parity, lib_parity = {}, 0, 0.0, 0.0, None, {}, {}
        for name, n, k in PROJECTIONS:
            packed = quantize(torch.randn(n, k, generator=gen, device=device) * 0.02)
            resident = backend.upload_linear(packed, dtype=torch.float16, device=device)
            del packed
            plan = resident.prepare(tokens=m)
            route = plan.route
            x = torch.randn(m, k, generator=gen, device=device).half()
            out = torch.empty(m, n, dtype=torch.float16, device=device)
            ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device) if plan.workspace_bytes else None
            kw = {} if ws is None else {"workspace": ws}
            t = event_time(lambda: plan.run(x, out=out, **kw), steps, warmup, stream)
            fused_us, fused_out = None, None
            if route in ("venturi-q4-dense", "venturi-q8-dense"):  # the fused kernel on the same weights, for comparison
                fused = resident.prepare(tokens=m, route="mfma")
                fused_out = torch.empty_like(out)
                fused_us = round(event_time(lambda: fused.run(x, out=fused_out), steps, warmup, stream) * 1e6, 1)
                plan.run(x, out=out, **kw)
            if codec == "w8a16":
                ref = torch.empty_like(out)
                resident.prepare(tokens=m, route="exact").run(x, out=ref)
            else:
                dense = torch.empty(n, k, dtype=torch.float16, device=device)
                resident._payload.decode(out=dense)
                ref = torch.nn.functional.linear(x, dense)
                del dense
            torch.cuda.synchronize(device)
            # `parity` is the hand-written kernel's (the roofline's); the library
            # route's own agreement is kept beside it.
            parity[name] = compact(agreement(out if fused_out is None else fused_out, ref))
            if fused_out is not None:
                lib_parity[name] = compact(agreement(out, ref))
            flops = 2 * m * n * k
            total_flops += flops
            total_s += t
            stages[name] = {"us": round(t * 1e6, 1), "TFLOP/s": round(flops / t / 1e12, 1),
                            "frac_fp16_peak": round(flops / t / 1e12 / FP16_PEAK_TFLOPS, 4)}
            if fused_us is not None:
                stages[name]["fused_mfma_us"] = fused_us
            fused_s += t if fused_us is None else fused_us / 1e6
            del resident, plan, x, out, ref, ws, fused_out
        tf = total_flops / total_s / 1e12
        fused_tf = total_flops / fused_s / 1e12
        kernel = "q8_prefill" if codec == "w8a16" else "row_prefill"
        library = {"venturi-q4-dense": "row_decode + hipBLASLt GEMM",
                   "venturi-q8-dense": "q8_split + hipBLASLt GEMM (2K)"}.get(route)
        sections[codec] = {"route": route, "TFLOP/s": round(tf, 1),
                           # The roofline is the hand-written matrix-core kernel's; the library
                           # route the auto plan takes at this size is reported beside it.
                           "roofline": {"bound": "mfma", "kernel": kernel + " (hand-written fp16 MFMA)",
                                        "achieved": round(fused_tf, 1), "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                        "frac": round(fused_tf / FP16_PEAK_TFLOPS, 4)},
                           **({"library_route": {"kernel": library, "note": "the auto route at 2048 tokens (vendor "
                                                 "GEMM over a decoded shadow), for comparison",
                                                 "TFLOP/s": round(tf, 1), "frac": round(tf / FP16_PEAK_TFLOPS, 4),
                                                 "parity": compact(merge_agreement(lib_parity.values()))}}
                              if library else {}),
                           "parity": {"kernel": kernel,
                                      "against": "canonical-order route" if codec == "w8a16" else
                                      "decoded fp16 weights + torch fp16 linear (the reference's W4A16 path)",
                                      "summary": compact(merge_agreement(parity.values())),
                                      "per_projection": parity},
                           "stages": stages}
    return {"workload": "fp16-activation prefill GEMMs at the config-2 shapes, M=2048", **sections}


# ---------------------------------------------------------------- Q4 / Q5 / Q6 decode


def q4_decode(backend, device, steps, warmup, copy_mb):
    """The metric's Q4 leg at M <= 16: the config-2 projection set with weights
    packed to q4_g64_fp16 (the W4A16 contract, plan route auto), M in {1,4,8,16}.

    Same method as the Q8 decode timing: per (projection, M), `steps` launches
    rotating >= `copy_mb` MB of independent weight copies captured in one HIP
    graph, replayed between one pair of events (per-launch durations), and the
    whole job as one graph (`GB/s`); algorithmic bytes per launch =
    codes N*Kp/2 + scales N*(Kp/64)*2 + activations M*K*2 + outputs M*N*2.
    """
    copies = []
    for i, (name, n, k) in enumerate(PROJECTIONS):
        count = max(2, -(-int(copy_mb * 1e6) // q4_launch_bytes(0, n, k)))
        residents = []
        for c in range(count):
            gen = torch.Generator(device=device).manual_seed(5000 + 1000 * c + i)
            w = torch.randn(n, k, generator=gen, device=device, dtype=torch.float32) * 0.02
            packed = backend.quantize_q4(w)
            del w
            residents.append(backend.upload_linear(packed, dtype=torch.float16, device=device))
            del packed
        copies.append(residents)
    gen = torch.Generator(device=device).manual_seed(17)
    xs = {m: {k: torch.randn(m, k, generator=gen, device=device).half() for k in {p[2] for p in PROJECTIONS}}
          for m in TOKENS}
    groups, route = {}, None
    for m in TOKENS:
        for pi, (name, n, k) in enumerate(PROJECTIONS):
            plans = [r.prepare(tokens=m) for r in copies[pi]]
            route = plans[0].route
            groups[(m, name)] = rotated_group(plans, xs[m][k], torch.empty(m, n, dtype=torch.float16, device=device),
                                              steps)
    seconds, wall, same = graph_timing(groups, steps, warmup, device)
    detail, total_bytes = {}, 0
    for m in TOKENS:
        for name, n, k in PROJECTIONS:
            t = seconds[(m, name)]
            b = steps * q4_launch_bytes(m, n, k)
            total_bytes += b
            detail[f"{name}_m{m}"] = {"us": round(t / steps * 1e6, 2), "GB/s": round(b / t / 1e9, 1)}
    achieved = total_bytes / sum(seconds.values()) / 1e9
    return {
        "workload": "config-2 projection set with q4_g64_fp16 weights (W4A16 contract), M in {1,4,8,16}",
        "route": route,
        "GB/s": round(total_bytes / wall / 1e9, 1),
        "roofline": {"bound": "hbm", "kernel": "row_decode_gemm (fp16 MFMA, W4A16 contract)", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4)},
        "weight_copies": {p[0]: len(c) for p, c in zip(PROJECTIONS, copies)},
        "graph_equals_eager": same,
        "per_launch": detail,
    }


def row_codec_decode(backend, device, steps, warmup, copy_mb, bits_list=(5, 6)):
    """Q5/Q6 row codecs (q5_g64 / q6_g64) at the config-2 shapes and M in {1, 4, 8, 16}:
    the W5A16 / W6A16 contract GEMM over tiled decode copies (`q5.tile_row_codec`,
    `venturi_row_tiled_run`, with exchange slots where K is split).

    Planes are synthetic bytes (random low nibbles and high bits, fp16 scales in
    [1e-4, 1e-2)); per (projection, M) `steps` launches rotate over >= `copy_mb`
    MB of copies inside one HIP graph; the whole job is one graph (GB/s).
    Algorithmic bytes per launch = N*Kp/2 + N*Kp*hb/8 + N*(Kp/64)*2 + M*K*2 + M*N*2.
    """
    from venturi_amd.q5 import tile_row_codec

    lib = backend._native
    stream = torch.cuda.current_stream(device)
    gen = torch.Generator(device=device).manual_seed(23)
    result = {"workload": "config-2 projection set with q5_g64 / q6_g64 planes (tiled decode copies), M in {1,4,8,16}",
              "kernel": "row_decode_gemm (fp16 MFMA, W*A16 contract, tiled copy)"}
    for bits in bits_list:
        hb = bits - 4

        def nbytes(m, n, k):
            padded = padded_k(k)
            return n * padded // 2 + n * padded * hb // 8 + n * (padded // 64) * 2 + m * k * 2 + m * n * 2

        copies = []
        for name, n, k in PROJECTIONS:
            padded = padded_k(k)
            count = max(2, -(-int(copy_mb * 1e6) // nbytes(0, n, k)))
            planes = []
            for _ in range(count):
                codes = torch.randint(0, 256, (n, padded // 2), dtype=torch.uint8, device=device, generator=gen)
                high = torch.randint(0, 256, (n, padded * hb // 8), dtype=torch.uint8, device=device, generator=gen)
                scales = (torch.rand(n, padded // 64, device=device, generator=gen) * 0.0099 + 1e-4).half()
                planes.append(tile_row_codec(codes, high, scales, bits))
                del codes, high, scales
            copies.append(planes)
        xs = {m: {k: torch.randn(m, k, generator=gen, device=device).half() for k in {p[2] for p in PROJECTIONS}}
              for m in TOKENS}
        groups = {}
        for m in TOKENS:
            for pi, (name, n, k) in enumerate(PROJECTIONS):
                size = int(lib.venturi_q4_tiled_workspace_bytes(m, n, k))
                slot = None
                if size:
                    slot = torch.empty(size, dtype=torch.uint8, device=device)
                    backend._check(lib.venturi_q4_tiled_workspace_init(slot.data_ptr(), size, stream.cuda_stream))
                out = torch.empty(m, n, dtype=torch.float16, device=device)

                def launch(r, out, m=m, n=n, k=k, pi=pi, slot=slot):
                    codes, high, scales = copies[pi][r % len(copies[pi])]
                    backend._check(lib.venturi_row_tiled_run(
                        xs[m][k].data_ptr(), codes.data_ptr(), high.data_ptr(), scales.data_ptr(), out.data_ptr(),
                        m, n, k, padded_k(k), bits, 0, None if slot is None else slot.data_ptr(),
                        0 if slot is None else slot.numel(), torch.cuda.current_stream(device).cuda_stream))

                def run(reps, launch=launch, out=out):
                    for r in range(reps):
                        launch(r, out)

                def verify(launch=launch, out=out):
                    ref = torch.empty_like(out)
                    launch(steps - 1, ref)
                    torch.cuda.synchronize(device)
                    return torch.equal(ref.view(torch.int16), out.view(torch.int16))

                groups[(m, name)] = (run, verify)
        seconds, wall, same = graph_timing(groups, steps, warmup, device)
        detail, total_bytes = {}, 0
        for m in TOKENS:
            for name, n, k in PROJECTIONS:
                t = seconds[(m, name)]
                b = steps * nbytes(m, n, k)
                total_bytes += b
                detail[f"{name}_m{m}"] = {"us": round(t / steps * 1e6, 2), "GB/s": round(b / t / 1e9, 1)}
        achieved = total_bytes / sum(seconds.values()) / 1e9
        result[f"q{bits}"] = {
            "GB/s": round(total_bytes / wall / 1e9, 1),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4)},
            "graph_equals_eager": same,
            "per_launch": detail,
        }
        del copies, groups
    return result


def codecs(backend, device, steps, warmup):
    """Row-codec pack and unpack on the device at the gate+up shape [34816 x 5120]:
    Q8 and Q4 packers from fp16 weights (`venturi_q8_pack_run`, `venturi_q4_pack_run`,
    bytes = fp16 read + codes and scales written), the Q4 row decoder to fp16
    (`venturi_row_dequant_rows`, planes read + fp16 written) and the Q8 embedding
    row gather (`venturi_q8_embedding_run`, 4096 ids). Each runs `steps` times
    back to back between one pair of events; inputs resident, outputs preallocated.
    """
    lib = backend._native
    n, k = 34816, 5120
    padded = padded_k(k)
    gen = torch.Generator(device=device).manual_seed(29)
    w = (torch.randn(n, k, generator=gen, device=device) * 0.02).half()
    c8 = torch.empty(n, padded, dtype=torch.int8, device=device)
    s8 = torch.empty(n, padded // 32, dtype=torch.float16, device=device)
    c4 = torch.empty(n, padded // 2, dtype=torch.uint8, device=device)
    s4 = torch.empty(n, padded // 64, dtype=torch.float16, device=device)
    dense = torch.empty(n, k, dtype=torch.float16, device=device)
    ids = torch.randint(0, n, (4096,), generator=gen, device=device, dtype=torch.int64)
    emb = torch.empty(4096, k, dtype=torch.float16, device=device)
    stream = torch.cuda.current_stream(device)
    s = stream.cuda_stream
    calls = {
        "q8_pack": (lambda: lib.venturi_q8_pack_run(w.data_ptr(), c8.data_ptr(), s8.data_ptr(), n, k, padded, 0, s),
                    n * k * 2 + n * padded + n * (padded // 32) * 2),
        "q4_pack": (lambda: lib.venturi_q4_pack_run(w.data_ptr(), c4.data_ptr(), s4.data_ptr(), n, k, padded, 0, s),
                    n * k * 2 + n * padded // 2 + n * (padded // 64) * 2),
        "q4_row_decode": (lambda: lib.venturi_row_dequant_rows(c4.data_ptr(), None, s4.data_ptr(), dense.data_ptr(), 0, n,
                                                               k, padded, 4, s),
                          n * padded // 2 + n * (padded // 64) * 2 + n * k * 2),
        "q8_embedding": (lambda: lib.venturi_q8_embedding_run(c8.data_ptr(), s8.data_ptr(), ids.data_ptr(),
                                                              emb.data_ptr(), 4096, n, k, padded, 0, s),
                         4096 * (padded + (padded // 32) * 2 + 8 + k * 2)),
    }
    out = {"workload": "device row-codec pack/unpack at [34816 x 5120] (fp16 source), embedding of 4096 rows"}
    for name, (fn, nbytes) in calls.items():
        t = event_time(lambda: backend._check(fn()), steps, warmup, stream)
        out[name] = {"us": round(t * 1e6, 1), "GB/s": round(nbytes / t / 1e9, 1),
                     "frac_hbm": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}
    return out


# ---------------------------------------------------------------- config 4


def moe_reference(x, ids, scores, dense_gu, dense_dn):
    """routed_experts (flash_next_moe.py:139-161) over fp16(q*s) expert weights on this GPU:
    ascending experts, fp16 linear with fp32 accumulation, fp16 SiLU*up, fp16 score
    multiply and index_add."""
    out = torch.zeros_like(x)
    inter = dense_gu[0].shape[0] // 2
    for e in range(len(dense_gu)):
        positions, tokens = torch.where((ids == e).T)
        if tokens.numel() == 0:
            continue
        gu = torch.nn.functional.linear(x[tokens], dense_gu[e])
        gate, up = gu[:, :inter], gu[:, inter:]
        h = torch.nn.functional.silu(gate) * up
        y = torch.nn.functional.linear(h, dense_dn[e])
        out.index_add_(0, tokens, y * scores[tokens, positions, None])
    return out


def moe_w4a16(backend, device, steps, warmup, cpu_seconds):
    """Config 4: routed-expert Q4 W4A16 MoE, 128 experts, H 2048, I 768, 512 tokens top-8.

    Expert weights N(0, 0.02) packed on the device with quantize_q4_rtn
    arithmetic; x fp16 N(0, 1); per token 8 distinct ids from a seeded
    randperm(128); scores = softmax of 8 seeded N(0, 1) logits (fp32 -> fp16).
    Two independent banks (2 x 321 MB) alternate so that no step is served
    from the 256 MB Infinity Cache. One step = routing + gate/up GEMM with
    SiLU*up + down GEMM with the score + ordered combine (three launches: the gate/up launch
    routes its experts itself at this pair count).
    Algorithmic bytes per step = expert planes + x + out + ids + scores;
    FLOPs = 2 * pairs * (2I*H + H*I). Parity against the reference's routed
    expert loop run with torch on this GPU (fp16(q*s) weights, fp16 linear).
    """
    from venturi_amd.moe import MoEGeometry, Q4ExpertBank

    g = MoEGeometry(2048, 128, 8, 768)
    tokens = 512
    banks, sample_planes, dense_gu, dense_dn = [], [], [], []
    for copy in range(2):
        experts = []
        for e in range(g.num_experts):
            gen = torch.Generator(device=device).manual_seed(100_000 * copy + e)
            gu = backend.quantize_q4(torch.randn(2 * g.intermediate_size, g.hidden_size, generator=gen, device=device) * 0.02)
            dn = backend.quantize_q4(torch.randn(g.hidden_size, g.intermediate_size, generator=gen, device=device) * 0.02)
            experts.append((gu, dn))
        banks.append(Q4ExpertBank.upload(backend, g, experts, device=device))
        if copy == 0:
            sample_planes = [(gu.codes.cpu(), gu.scales.cpu(), dn.codes.cpu(), dn.scales.cpu()) for gu, dn in experts[:16]]
            for gu, dn in experts:
                for w, rows, cols, dest in ((gu, 2 * g.intermediate_size, g.hidden_size, dense_gu),
                                            (dn, g.hidden_size, g.intermediate_size, dense_dn)):
                    d = torch.empty(rows, cols, dtype=torch.float16, device=device)
                    backend._check(backend._native.venturi_row_dequant_rows(
                        w.codes.data_ptr(), None, w.scales.data_ptr(), d.data_ptr(), 0, rows, cols, w.padded_k, 4,
                        torch.cuda.current_stream(device).cuda_stream))
                    dest.append(d)
        del experts
    cpu_gen = torch.Generator().manual_seed(4)
    ids = torch.stack([torch.randperm(g.num_experts, generator=cpu_gen)[: g.top_k] for _ in range(tokens)])
    scores = torch.softmax(torch.randn(tokens, g.top_k, generator=cpu_gen), -1).half()
    x = torch.randn(tokens, g.hidden_size, generator=cpu_gen).half()
    xd, idsd, scoresd = x.to(device), ids.to(device), scores.to(device)
    plans = [b.prepare(tokens=tokens) for b in banks]
    workspace = torch.empty(plans[0].workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty(tokens, g.hidden_size, dtype=torch.float16, device=device)
    stream = torch.cuda.current_stream(device)
    counter = [0]

    def step():
        plans[counter[0] % 2].run(xd, idsd, scoresd, out=out, workspace=workspace)
        counter[0] += 1

    step_s = event_time(step, steps, warmup, stream)
    plans[0].run(xd, idsd, scoresd, out=out, workspace=workspace)
    ref = moe_reference(xd, idsd, scoresd, dense_gu, dense_dn)
    torch.cuda.synchronize(device)
    parity = compact(agreement(out, ref))
    del dense_gu, dense_dn, ref
    pairs = tokens * g.top_k
    nbytes = banks[0].storage_nbytes + 2 * tokens * g.hidden_size * 2 + pairs * (8 + 2)
    flops = 2 * pairs * (2 * g.intermediate_size * g.hidden_size + g.hidden_size * g.intermediate_size)
    gbs = nbytes / step_s / 1e9
    result = {
        "workload": "config4: Q4 W4A16 routed experts, 128 experts, H 2048, I 768, 512 tokens top-8",
        "us_per_step": round(step_s * 1e6, 2),
        "GB/s": round(gbs, 1),
        "TFLOP/s": round(flops / step_s / 1e12, 2),
        "tokens_per_s": round(tokens / step_s, 1),
        "bytes_per_step": nbytes,
        "flops_per_step": flops,
        "roofline": {"bound": "hbm", "kernel": "q4_grouped", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "fp16_mfma_frac": round(flops / step_s / 1e12 / FP16_PEAK_TFLOPS, 4)},
        "parity": {"against": "routed_experts loop with torch fp16 linear over fp16(q*s) weights on this GPU",
                   **parity},
    }
    if cpu_seconds > 0:
        from oracle.cpu_path import CpuRoutedExperts, cpu_threads, q4_fp32_weight, time_calls

        threads = cpu_threads()
        sample = list(range(len(sample_planes)))
        gate_up = [q4_fp32_weight(p[0], p[1], g.hidden_size) for p in sample_planes]
        down = [q4_fp32_weight(p[2], p[3], g.intermediate_size) for p in sample_planes]
        runner = CpuRoutedExperts(gate_up, down)
        reps, elapsed = time_calls([lambda: runner.run(x, ids, scores, sample)], cpu_seconds)
        full_s = elapsed / reps * g.num_experts / len(sample)
        result["cpu_baseline"] = {
            "value": round(nbytes / full_s / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"experts 0-15 of 128 ({reps} repetitions, {elapsed:.1f} s), staged-fp32 cpu_expert path "
            f"with pre-materialised fp32 weights, scaled x8 to the full step ({full_s * 1e3:.1f} ms per step); "
            f"{cpu_description(threads)}",
        }
    del banks, plans
    return result


# ---------------------------------------------------------------- vocabulary head


def vocab_head(backend, device, steps, warmup, tokens_list=(1, 4, 16)):
    """The Q8 vocabulary head at the model's shape: vocab 248 320 x hidden 5120
    (1.35 GB of q8_g32_fp16 per token, larger than the Infinity Cache, so
    back-to-back launches stream from HBM), held once in the tiled layout
    (``residency="tiled"``) and run on the matrix-core decode route; `steps`
    launches per token count in one HIP graph between events. Algorithmic
    bytes per launch = N*Kp*(1+2/32) + M*K*2 + M*N*2. The canonical-order
    route (row-major planes) is timed at one token beside it.
    """
    vocab, hidden = 248320, 5120
    gen = torch.Generator(device=device).manual_seed(248320)
    packed = backend.quantize_q8(torch.randn(vocab, hidden, generator=gen, device=device) * 0.02)
    torch.cuda.empty_cache()
    resident = backend.upload_linear(packed, dtype=torch.float16, device=device, residency="tiled")
    result = {"workload": "Q8 vocabulary head 248320 x 5120 (tiled residency, one copy)",
              "resident_bytes": resident.storage_nbytes}
    xs = {m: torch.randn(m, hidden, generator=gen, device=device).half() for m in tokens_list}
    detail, total_b, total_s = {}, 0, 0.0
    for m in tokens_list:
        plan = resident.prepare(tokens=m)
        out = torch.empty(m, vocab, dtype=torch.float16, device=device)
        seconds, _, same = graph_timing({m: rotated_group([plan], xs[m], out, steps)}, steps, warmup, device)
        avg = seconds[m] / steps
        b = launch_bytes(m, vocab, hidden)
        total_b += b
        total_s += avg
        detail[f"m{m}"] = {"us": round(avg * 1e6, 2), "GB/s": round(b / avg / 1e9, 1), "graph_equals_eager": same}
    del resident
    torch.cuda.empty_cache()
    full = backend.upload_linear(packed, dtype=torch.float16, device=device)
    exact = full.prepare(tokens=1, route="exact")
    out = torch.empty(1, vocab, dtype=torch.float16, device=device)
    seconds, _, _ = graph_timing({"exact": rotated_group([exact], xs[1], out, steps)}, steps, warmup, device)
    ex = seconds["exact"] / steps
    detail["m1_exact_route"] = {"us": round(ex * 1e6, 2), "GB/s": round(launch_bytes(1, vocab, hidden) / ex / 1e9, 1)}
    del full, packed
    torch.cuda.empty_cache()
    gbs = total_b / total_s / 1e9
    result["roofline"] = {"bound": "hbm", "kernel": "q8_tiled_lds / q8_tiled_decode (fp16 MFMA)",
                          "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(gbs / HBM_PEAK_GBS, 4)}
    result["per_launch"] = detail
    return result


# ---------------------------------------------------------------- config 5


def model_decode(backend, device, steps, warmup, batches=(1, 8, 32)):
    """Config 5: 64 decoder layers x the config-2 projections, all resident (256 Q8 matrices).

    One step chains, per layer: h -> QKV; a seeded fp16 [B, 6144] -> o_proj;
    h -> gate+up fused with SiLU*up (the native runtime's SwiGLU arithmetic
    in the projection's epilogue) -> down -> next h. Each matrix is resident
    once, in the tiled layout its decode kernel reads (no row-major copy). The 256 launches of a
    step are captured once in a HIP graph (checked bit-for-bit against an
    eager step) and replayed. Projection-only tokens/s = B / step time; GB/s counts the
    projections' algorithmic bytes (weights + activations + outputs).
    """
    layers = 64
    matrices = []
    for layer in range(layers):
        row = []
        for i, (name, n, k) in enumerate(PROJECTIONS):
            gen = torch.Generator(device=device).manual_seed(7_000_000 + 16 * layer + i)
            w = torch.randn(n, k, generator=gen, device=device) * 0.02
            # One resident copy per matrix, in the layout its decode kernel reads.
            residency = "tiled-paired" if name == "gate_up" else "tiled"
            row.append(backend.upload_linear(backend.quantize_q8(w), dtype=torch.float16, device=device,
                                             residency=residency))
            del w
        matrices.append(row)
    torch.cuda.synchronize(device)
    weight_bytes = sum(r.storage_nbytes for row in matrices for r in row)
    inter = PROJECTIONS[2][1] // 2
    results = {}
    for b in batches:
        plans = [[r.prepare_swiglu(tokens=b) if i == 2 else r.prepare(tokens=b) for i, r in enumerate(row)]
                 for row in matrices]
        gen = torch.Generator(device=device).manual_seed(b)
        h0 = torch.randn(b, 5120, generator=gen, device=device).half()
        o_in = torch.randn(b, 6144, generator=gen, device=device).half()
        h = [h0.clone(), torch.empty_like(h0)]
        qkv = torch.empty(b, PROJECTIONS[0][1], dtype=torch.float16, device=device)
        o = torch.empty(b, PROJECTIONS[1][1], dtype=torch.float16, device=device)
        act = torch.empty(b, inter, dtype=torch.float16, device=device)

        def step():
            h[0].copy_(h0)
            for layer in range(layers):
                p = plans[layer]
                cur, nxt = h[layer % 2], h[(layer + 1) % 2]
                p[0].run(cur, out=qkv)
                p[1].run(o_in, out=o)
                p[2].run(cur, out=act)
                p[3].run(act, out=nxt)

        step()
        torch.cuda.synchronize(device)
        eager = h[layers % 2].clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        graph.replay()
        torch.cuda.synchronize(device)
        same = bool(torch.equal(h[layers % 2].view(torch.int16), eager.view(torch.int16)))
        step_s = event_time(graph.replay, steps, warmup, torch.cuda.current_stream(device))
        step_bytes = layers * sum(launch_bytes(b, n, k) for _, n, k in PROJECTIONS)
        results[f"B{b}"] = {
            "ms_per_step": round(step_s * 1e3, 4),
            "tokens_per_s": round(b / step_s, 1),
            "GB/s": round(step_bytes / step_s / 1e9, 1),
            "frac_hbm": round(step_bytes / step_s / 1e9 / HBM_PEAK_GBS, 4),
            "route": plans[0][0].route,
            "graph_equals_eager": same,
        }
        del plans, graph
    del matrices
    return {
        "workload": "config5: 64 layers x config-2 Q8 projections resident, chained per step (HIP graph, gate+up fused with SiLU*up)",
        "weight_bytes": weight_bytes,
        "batches": results,
    }


# ---------------------------------------------------------------- main


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, ROOT)
    from venturi_amd import create_backend

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    backend = create_backend("hip")
    only = set(args.only.split(",")) if args.only else None

    def wanted(name, skip=False):
        return (name in only) if only is not None else not skip

    if only is None or "config2" in only:
        result, copies = config2(backend, device, args)
        cpu_copies = None if args.no_cpu else [[r[0]] for r in copies]
        del copies
    else:  # a section run (counter collection): no headline metric
        result, cpu_copies = {"sections": sorted(only)}, None
    torch.cuda.empty_cache()
    if wanted("config1"):
        log("config 1: 4096 x 4096 at one token")
        result["config1"] = config1(backend, device, args.steps, args.warmup, args.copy_mb)
    if wanted("head"):
        log("vocabulary head 248320 x 5120")
        result["vocab_head"] = vocab_head(backend, device, args.steps, args.warmup)
    if wanted("q4", args.no_q4):
        log("Q4 W4A16 decode at the config-2 shapes")
        result["q4_decode"] = q4_decode(backend, device, args.steps, args.warmup, args.copy_mb)
    if wanted("q56", args.no_q4):
        log("Q5/Q6 row-codec decode at the config-2 shapes")
        result["q56_decode"] = row_codec_decode(backend, device, args.steps, args.warmup, args.copy_mb)
    torch.cuda.empty_cache()
    if wanted("codecs"):
        log("row-codec pack/unpack on the device")
        result["codecs"] = codecs(backend, device, max(args.steps // 2, 3), 2)
    if wanted("a8dec", args.no_prefill):
        log("A8 decode at the config-2 shapes")
        result["a8_decode"] = a8_decode(backend, device, args.steps, args.warmup, args.copy_mb)
    torch.cuda.empty_cache()
    if wanted("a8", args.no_prefill):
        log("config-3 A8 prefill")
        result["prefill_a8"] = prefill_a8(backend, device, max(args.steps // 2, 3), 2, 0 if args.no_cpu else 6.0)
    if wanted("a16", args.no_prefill):
        log("fp16-activation prefill GEMMs (W8A16, W4A16)")
        result["prefill_a16"] = prefill_a16(backend, device, max(args.steps // 2, 3), 2)
    torch.cuda.empty_cache()
    if wanted("moe", args.no_moe):
        log("config-4 routed-expert MoE")
        result["moe_w4a16"] = moe_w4a16(backend, device, max(args.steps, 10), 3, 0 if args.no_cpu else 4.0)
    torch.cuda.empty_cache()
    if wanted("model", args.no_model):
        log("config-5 64-layer streaming decode")
        result["model_decode"] = model_decode(backend, device, max(args.steps // 4, 3), 2)
    if cpu_copies is not None:
        log("CPU baseline (reference CPU path)")
        result["cpu_baseline"] = cpu_baseline(cpu_copies, args.cpu_seconds)
    print(json.dumps(result if args.full else shorten(result)), flush=True)


if __name__ == "__main__":
    main()
