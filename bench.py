#!/usr/bin/env python3
"""Benchmark of the FP8 projection path on one MI355X.

    python bench.py [--config C2] [--steps K] [--warmup W] [--no-cpu] [--no-others]

A "step" is one pass of the hot path over one batch of synthetic input:
per-token quantization of every projection input, the FP8 GEMMs with fused
epilogues, and the re-quantization of GELU/GLU outputs. The headline workload is
BASELINE configs[1] (C2: GR00T-style DiT action head, M=16, 4 flow-matching
steps per timed unit), reported in GB/s of algorithmic HBM traffic; C1, C3, C4
and C5 are measured in the same run and reported under "configs".

Timing: K steps are captured into one HIP graph (inputs already resident in HBM,
weights rotating through a pool larger than the 256 MB Infinity Cache for
M <= 64) and replayed once between synchronizations, after W warm-up steps.
The dominant kernel's average duration is measured separately with HIP events
around a graph of back-to-back launches of that kernel alone, on the stream it
runs on, and gives the "roofline" object.

The CPU baseline runs the reference's PyTorch CPU FP8 path (oracle/cpu_path.py)
on the host cores: whole C2 units, repeated until about 10 s of CPU time.
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
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
FP8_PEAK_TFLOPS = 5000.0     # MI355X dense FP8 MFMA, TFLOP/s
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "FP8 linear TFLOP/s (% of MI355X FP8 MFMA peak) + GB/s for M<=64; p50 us/call"


def _log(*a):
    print(*a, file=sys.stderr, flush=True)


def capture(fn, n, stream):
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(n):
            fn(i)
    return g


def time_graph(g, reps=1):
    """Replay g `reps` times; returns (event ms, wall ms) over all replays."""
    import torch
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(reps):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return e0.elapsed_time(e1), (t1 - t0) * 1e3


def measure(wl, steps, warmup, kernel_launches=64):
    """Returns per-step and dominant-kernel timings of one workload."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # eager warm-up on the capture stream (workspaces, code objects)
        for _ in range(2):
            wl.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    gw = capture(lambda i: wl.step(), max(warmup, 1), side)
    gk = capture(lambda i: wl.step(), steps, side)
    gd = capture(lambda i: wl.dominant_call(i), kernel_launches, side)
    time_graph(gw)
    ev_ms, wall_ms = time_graph(gk)
    time_graph(gd)  # warm
    samples = [time_graph(gd)[0] / kernel_launches for _ in range(5)]
    samples.sort()
    kern_ms = samples[len(samples) // 2]
    return dict(step_ms=ev_ms / steps, wall_step_ms=wall_ms / steps, kernel_ms=kern_ms)


def measure_calls(wl, launches):
    """p50 µs of every call of the path on its own (graph of back-to-back calls,
    weights rotating as in the step), with TFLOP/s, GB/s and both roofline
    fractions (the C4 qkv / o projections sit near the ridge point)."""
    import torch
    out = []
    side = torch.cuda.Stream()
    for c in wl.calls():
        side.wait_stream(torch.cuda.current_stream())
        g = capture(lambda i: c.fn(i), launches, side)
        time_graph(g)
        us = sorted(time_graph(g)[0] / launches * 1e3 for _ in range(5))[2]
        w = c.work
        shape = f"{w.M}x{w.N}x{w.K}" + (f" {w.act}" if w.act else "") if c.kind == "gemm" else f"{w[0]}x{w[1]}"
        tf = c.flops / us / 1e6
        gbs = c.bytes / us / 1e3
        out.append({"call": c.name, "kind": c.kind, "shape": shape, "us_p50": round(us, 3),
                    "tflops": round(tf, 2), "gbs": round(gbs, 1), "frac_mfma": round(tf / FP8_PEAK_TFLOPS, 4),
                    "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
        del g
    return out


def summarize(wl, m):
    step_s = m["step_ms"] * 1e-3
    d = wl.dominant_gemm
    k_s = m["kernel_ms"] * 1e-3
    res = {
        "title": wl.title,
        "bound": wl.bound,
        "us_per_step": round(m["step_ms"] * 1e3, 3),
        "tflops": round(wl.flops / step_s / 1e12, 2),
        "gbs": round(wl.bytes / step_s / 1e9, 1),
        "gemm_gflop_per_step": round(wl.flops / 1e9, 3),
        "bytes_per_step": wl.bytes,
        "dominant": {
            "kernel": f"{d.name} {d.M}x{d.N}x{d.K}" + (f" {d.act}" if d.act else ""),
            "us": round(m["kernel_ms"] * 1e3, 3),
            "tflops": round(d.flops / k_s / 1e12, 2),
            "gbs": round(d.bytes / k_s / 1e9, 1),
            "frac_mfma": round(d.flops / k_s / 1e12 / FP8_PEAK_TFLOPS, 4),
            "frac_hbm": round(d.bytes / k_s / 1e9 / HBM_PEAK_GBS, 4),
        },
    }
    res["frac_step"] = round(res["gbs"] / HBM_PEAK_GBS, 4) if wl.bound == "hbm" else \
        round(res["tflops"] / FP8_PEAK_TFLOPS, 4)
    return res


def measure_producers(dev, launches=32):
    """The kernels around the projections: the pre-norm producer (residual
    update + LayerNorm + adaLN + per-token quant) at the C5 and C2 shapes, the
    QKV split / Wan QKV consumers, the MoE router and routed activation, and
    attention with the fused FP8 output row: µs per call (graph of back-to-back
    calls, median of 5), GB/s of algorithmic bytes against the 8 TB/s roofline
    and, for attention, TFLOP/s against the 2.5 PFLOP/s bf16 peak."""
    import torch
    from instinctflash_amd.workloads import CONSUMERS, PRODUCERS, NormQuant
    res = {}
    jobs = [(f"residual_norm_quant {key}", lambda M=M, D=D: NormQuant(dev, M, D)) for key, (M, D) in PRODUCERS.items()]
    jobs += [(f"{cls.__name__} {key}", lambda cls=cls: cls(dev)) for key, cls in CONSUMERS.items()]
    for key, make in jobs:
        p = make()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            p.step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = capture(lambda i: p.step(i), launches, side)
        time_graph(g)
        us = sorted(time_graph(g)[0] / launches * 1e3 for _ in range(5))[2]
        gbs = p.bytes / us / 1e3
        res[key] = {"kernel": p.title, "us": round(us, 3), "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                    "bytes": p.bytes}
        if hasattr(p, "flops"):  # bf16 matrix-core work (attention)
            tf = p.flops / us / 1e6
            res[key].update(tflops=round(tf, 2), frac_bf16_mfma=round(tf / BF16_PEAK_TFLOPS, 4))
        _log(f"[bench] {key}: {p.title}: {us:.2f} us, {gbs:.0f} GB/s")
    return res


def measure_engine(dev, reps=5):
    """The pi05 action expert end to end on these kernels (reference
    engines/pi05/engine.py:212-245): 10 Euler steps x 18 layers over an
    800-row prefix cache, random weights of the architecture, one captured
    graph; ms per 50-action chunk (median of `reps` replays)."""
    import torch
    from instinctflash_amd.pi05 import Pi05Expert, random_weights
    w = random_weights(dev, layers=18, steps=10, seed=0)
    eng = Pi05Expert(w, dev, smax=832)
    g = torch.Generator().manual_seed(1)
    eng.kc[:, :800] = torch.randn(18, 800, 1, 256, generator=g).half().to(dev)
    eng.vc[:, :800] = torch.randn(18, 800, 1, 256, generator=g).half().to(dev)
    eng.set_prefix(800)
    eng.noise.copy_(torch.randn(eng.chunk, 32, generator=g))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eng.forward()
    torch.cuda.current_stream().wait_stream(side)
    graph = capture(lambda i: eng.forward(), 1, side)
    time_graph(graph)
    ms = sorted(time_graph(graph)[0] for _ in range(reps))[reps // 2]
    launches = 10 * (2 + 18 * 8)
    _log(f"[bench] pi05 expert: {ms:.3f} ms per 50-action chunk ({launches} kernels + torch addmm)")
    return {"workload": "pi05 action expert, 10 steps x 18 layers, prefix 800, chunk 50 (random weights)",
            "ms_per_chunk": round(ms, 4), "kernels_per_chunk": launches}


def probe(wl, dev, launches=20, copy_bytes=1 << 30):
    """Counter-run helper: the dominant kernel alone, then a plain copy of known
    size (the calibration for FETCH_SIZE / WRITE_SIZE), each `launches` times."""
    import torch
    for _ in range(2):
        wl.step()  # inputs of the dominant call, workspaces, code objects
    torch.cuda.synchronize()
    for i in range(launches):
        wl.dominant_call(i)
    torch.cuda.synchronize()
    src = torch.empty(copy_bytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    src.fill_(1)
    for _ in range(launches):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"probe": wl.key, "dominant": wl.dominant, "launches": launches, "copy_bytes": copy_bytes}))


def cpu_baseline(min_seconds=10.0):
    """Reference CPU FP8 path for one C2 unit (4 flow steps = 8 projections)."""
    import torch
    from oracle import cpu_path
    from instinctflash_amd.workloads import C2, Gemm, quant_bytes
    g = torch.Generator().manual_seed(0)
    M, D, FF = 16, 1536, 6144
    xs = [torch.randn((M, D), generator=g).to(torch.bfloat16) for _ in range(4)]
    w1 = torch.randn((FF, D), generator=g) * 0.02
    w2 = torch.randn((D, FF), generator=g) * 0.02
    res = torch.randn((M, D), generator=g).to(torch.bfloat16)
    q1, s1 = cpu_path.quant_rows(w1)
    q2, s2 = cpu_path.quant_rows(w2)
    cpu_path.c2_unit(xs, q1, s1, q2, s2, res)  # warm-up (oneDNN primitive creation)
    units, t0 = 0, time.perf_counter()
    while True:  # a bounded sample: whole units until ~min_seconds of CPU work
        cpu_path.c2_unit(xs, q1, s1, q2, s2, res)
        units += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds or units >= 100000:
            break
    dt /= units
    gemms = [Gemm("up", M, FF, D, act="gelu_tanh"), Gemm("down", M, D, FF, residual=True)]
    nbytes = 4 * (sum(x.bytes for x in gemms) + quant_bytes(M, D) + quant_bytes(M, FF))
    # second line: the same unit with dequantize-then-fp32-matmul (MKL) in place of _scaled_mm
    d1, d2 = q1.float() * s1[:, None], q2.float() * s2[:, None]
    cpu_path.c2_unit_fp32(xs, d1, d2, res)
    units32, t0 = 0, time.perf_counter()
    while True:
        cpu_path.c2_unit_fp32(xs, d1, d2, res)
        units32 += 1
        dt32 = time.perf_counter() - t0
        if dt32 >= min_seconds / 2 or units32 >= 100000:
            break
    dt32 /= units32
    return {"value": round(nbytes / dt / 1e9, 4), "unit": "GB/s", "cores": torch.get_num_threads(),
            "dequant_fp32_matmul": {"value": round(nbytes / dt32 / 1e9, 4), "unit": "GB/s",
                                    "seconds_per_unit": round(dt32, 6), "units_timed": units32,
                                    "sample": "same C2 units: per-token quant, dequantize, fp32 matmul (MKL), "
                                              "fp32 epilogue"},
            "kind": "port", "seconds_per_unit": round(dt, 4), "units_timed": units,
            "sample": f"{units} full C2 units (4 flow steps x [quant, 16x1536->6144 GELU, quant, 16x6144->1536 "
                      "+res]) via torch._scaled_mm (oneDNN) on the host CPU, reference GI decomposition",
            "cpu": _cpu_model(), "os_cpu_count": os.cpu_count()}


def measured_traffic(config):
    """(bytes per launch, file) from profiles/hbm_traffic_<config>.md, if committed."""
    import re
    f = ROOT / "profiles" / f"hbm_traffic_{config}.md"
    if not f.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch = (\d+)", f.read_text())
    return (int(m.group(1)), f"profiles/{f.name}") if m else None


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="C2", choices=["C1", "C2", "C3", "C4", "C5"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-others", action="store_true")
    ap.add_argument("--probe", action="store_true",
                    help="launch only the dominant kernel (20x, no graph) and a 1 GiB device copy (20x), "
                         "for rocprofv3 counter runs; prints nothing else")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the FP8 projection path has no multi-GPU step in this build "
              "(sharded, it would split each projection by output channels, one shard per GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from instinctflash_amd import _lib
    from instinctflash_amd.workloads import CONFIGS
    if not torch.cuda.is_available():
        print("bench.py needs the MI355X GPU", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    dev = torch.device("cuda:0")
    arch = torch.cuda.get_device_properties(0).gcnArchName
    if args.probe:
        probe(CONFIGS[args.config](dev), dev)
        return

    results = {}
    order = [args.config] + ([] if args.no_others else [k for k in CONFIGS if k != args.config])
    for key in order:
        wl = CONFIGS[key](dev)
        steps = args.steps if key == args.config else max(10, min(args.steps, 20))
        _log(f"[bench] {key}: {wl.title} (pool {wl.pool}, {steps} steps)")
        m = measure(wl, steps, args.warmup)
        results[key] = summarize(wl, m)
        results[key]["steps"] = steps
        results[key]["calls"] = measure_calls(wl, 32 if wl.bound == "hbm" else 8)
        if key == args.config:
            head = (wl, m)
        del wl
        torch.cuda.empty_cache()

    wl, m = head
    r = results[args.config]
    d = wl.dominant_gemm
    k_s = m["kernel_ms"] * 1e-3
    if wl.bound == "hbm":
        value, unit = r["gbs"], "GB/s"
        roof = {"bound": "hbm", "achieved": round(d.bytes / k_s / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    else:
        value, unit = r["tflops"], "TFLOP/s"
        roof = {"bound": "mfma", "achieved": round(d.flops / k_s / 1e12, 2), "peak": FP8_PEAK_TFLOPS,
                "unit": "TFLOP/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["traffic"] = None
    measured = measured_traffic(args.config)
    if measured is not None:
        # HBM bytes per launch of the dominant kernel from calibrated FETCH_SIZE /
        # WRITE_SIZE counter runs (summary and commands in the profiles/ file)
        roof["traffic"] = measured[0]
        roof["traffic_source"] = measured[1]
        roof["traffic_vs_algorithmic"] = round(measured[0] / d.bytes, 3)
    roof["algorithmic_bytes"] = d.bytes
    roof["kernel"] = r["dominant"]["kernel"]
    roof["kernel_us"] = r["dominant"]["us"]

    out = {
        "metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(m["step_ms"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8-e4m3 x fp8-e4m3 -> fp32 acc, bf16 out",
        "data": "synthetic (seeded torch.Generator on CPU, random-init weights quantized per channel)",
        "config": {"workload": f"{args.config}: {wl.title}", "M": d.M, "gpu": arch,
                   "timed_unit": "4 flow-matching steps" if wl.steps_per_unit > 1 else "one pass"},
        "roofline": roof,
    }
    if not args.no_others:
        out["producers"] = measure_producers(dev)
        out["engine"] = measure_engine(dev)
    if not args.no_cpu:
        _log("[bench] CPU baseline (reference CPU FP8 path, one C2 unit)")
        out["cpu_baseline"] = cpu_baseline()
    out["configs"] = results
    print(json.dumps(out))


if __name__ == "__main__":
    main()
