#!/usr/bin/env python3
"""Benchmark of the FP8 projection path on one MI355X.

    python bench.py [--config C5] [--steps K] [--warmup W] [--no-cpu] [--no-others]

A "step" is one pass of the hot path over one batch of synthetic input:
per-token quantization of every projection input, the FP8 GEMMs with fused
epilogues, and the re-quantization of GELU/GLU outputs. The headline workload is
the largest single-GPU configuration, C5 (Wan DiT block projections, M=8192),
reported in TFLOP/s of FP8 GEMM work; C1-C4 are measured in the same run and
reported under "configs", each with its own roofline and CPU baseline (C1/C2 in
GB/s of algorithmic HBM traffic: they are bandwidth-bound).

Timing: K steps are captured into one HIP graph (inputs already resident in HBM,
weights rotating through a pool larger than the 256 MB Infinity Cache for
M <= 64) and replayed once between synchronizations, after W warm-up steps.
The dominant kernel's average duration is measured separately with HIP events
around a graph of back-to-back launches of that kernel alone, on the stream it
runs on, and gives the "roofline" object.

The shader clock under the headline's dominant kernel is measured live: a
one-wave probe kernel (ifx_sclk_probe) on a second stream counts shader cycles
against the constant-rate wall clock while that kernel's graph replays.

The CPU baseline runs the reference's PyTorch CPU FP8 path (oracle/cpu_path.py)
on the host cores for every config: C1 and C2 whole, C3-C5 on a row sample
(the same calls with fewer tokens), extrapolated linearly in M and labelled so.
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
        with torch.cuda.stream(side):  # eager first call on the capture stream (its workspace)
            c.fn(0)
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


def measure_vendor(wl, calls, launches):
    """The vendor library on the same GEMM shapes: hipBLASLt FP8 through
    torch._scaled_mm (e4m3 x e4m3, per-token and per-channel fp32 scales,
    bf16 out, the reference's GEMM call: instinctflash/kernels/fp8.py:50-53),
    µs per call in a graph of back-to-back calls (median of 5), weights rotating
    through a pool of the workload's size as in the step. hipBLASLt fuses only
    the scales: no bias, activation, gate or residual, and a GLU projection
    writes both halves (2F columns), so its bytes are a lower bound of the
    reference path's. Returns None if this torch build lacks row-wise scaling."""
    import torch
    from instinctflash_amd.kernels import fp8 as F
    gemms = [c for c in wl.calls() if c.kind == "gemm"]
    ours = {c["call"]: c["us_p50"] for c in calls if c["kind"] == "gemm"}
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(7)
    side = torch.cuda.Stream()
    rows, ours_sum, vendor_sum = [], 0.0, 0.0
    for c in gemms:
        w = c.work
        a, sa = F.quant_rows(torch.randn((w.M, w.K), generator=g).to(torch.bfloat16).to(dev))
        pool = max(1, wl.pool)
        ws = [F.quantize_weight(torch.randn((w.N, w.K), generator=g) * 0.02, device=dev)] if pool == 1 else None
        if ws is None:
            base = F.quantize_weight(torch.randn((w.N, w.K), generator=g) * 0.02, device=dev)
            ws = [base] + [F.Fp8Weight(base.w.clone(), base.scale.clone()) for _ in range(pool - 1)]
        out = torch.empty((w.M, w.N), dtype=torch.bfloat16, device=dev)
        sa2 = sa.view(-1, 1)
        sws = [x.scale.view(1, -1) for x in ws]

        def fn(i, ws=ws, sws=sws, a=a, sa2=sa2, out=out):
            k = i % len(ws)
            torch._scaled_mm(a, ws[k].w.t(), scale_a=sa2, scale_b=sws[k], out_dtype=torch.bfloat16, out=out)
        try:
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                fn(0)
            torch.cuda.synchronize()
        except (RuntimeError, NotImplementedError) as exc:  # no row-wise FP8 in this build
            _log(f"[bench] hipBLASLt comparator unavailable: {exc}")
            return None
        gr = capture(fn, launches, side)
        time_graph(gr)
        us = sorted(time_graph(gr)[0] / launches * 1e3 for _ in range(5))[2]
        del gr, ws
        rows.append({"call": c.name, "shape": f"{w.M}x{w.N}x{w.K}", "us_p50": round(us, 3),
                     "tflops": round(w.flops / us / 1e6, 2), "ours_us_p50": ours.get(c.name)})
        vendor_sum += us
        ours_sum += ours.get(c.name, 0.0)
    torch.cuda.empty_cache()
    return {"library": "hipBLASLt via torch._scaled_mm (row-wise scales, bf16 out, no fused epilogue)",
            "calls": rows, "gemm_us_sum": round(vendor_sum, 2), "ours_gemm_us_sum": round(ours_sum, 2),
            "speedup_ours_vs_vendor": round(vendor_sum / ours_sum, 3) if ours_sum else None}


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


def roofline(wl, m):
    """Roofline object of the config's dominant kernel: algorithmic FLOPs (MFMA-
    bound configs) or bytes (HBM-bound) per launch / its mean launch time (HIP
    events around a graph of back-to-back launches on its own stream), against
    the MI355X peak; `traffic` = calibrated HBM bytes per launch from the
    committed profiles/hbm_traffic_<config>.md counter summary, when present."""
    d = wl.dominant_gemm
    k_s = m["kernel_ms"] * 1e-3
    if wl.bound == "hbm":
        roof = {"bound": "hbm", "achieved": round(d.bytes / k_s / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    else:
        roof = {"bound": "mfma", "achieved": round(d.flops / k_s / 1e12, 2), "peak": FP8_PEAK_TFLOPS,
                "unit": "TFLOP/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["traffic"] = None
    measured = measured_traffic(wl.key)
    if measured is not None:
        roof["traffic"] = measured[0]
        roof["traffic_source"] = measured[1]
        roof["traffic_vs_algorithmic"] = round(measured[0] / d.bytes, 3)
    roof["algorithmic_bytes"] = d.bytes
    roof["algorithmic_flops"] = d.flops
    roof["kernel"] = f"{d.name} {d.M}x{d.N}x{d.K}" + (f" {d.act}" if d.act else "")
    roof["kernel_us"] = round(m["kernel_ms"] * 1e3, 3)
    return roof


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


def measure_pi05(dev, reps=5):
    """The whole pi05 prediction on these kernels (instinctflash_amd/
    pi05_forward.py; the model of reference engines/pi05/engine.py): 3 camera
    views through the 27-layer SigLIP tower and the projector, the 18-layer
    Gemma-2B prefix over 816 rows (768 image + 48 prompt rows: config C3's M),
    and 10 Euler steps of the 18-layer action expert over the 50-action chunk,
    random weights, one captured graph; ms per chunk (median of `reps`
    replays). The reference publishes 51.85 ms for this forward on Jetson Thor
    (README.md:38)."""
    import torch
    from instinctflash_amd.pi05_forward import Pi05Dims, Pi05Forward, random_pi05
    d = Pi05Dims()
    fwd = Pi05Forward(random_pi05(d, dev, seed=0), dev)
    g = torch.Generator(device=dev).manual_seed(1)
    fwd.set_inputs(torch.rand(d.views, 3, 224, 224, generator=g, device=dev) * 2 - 1,
                   torch.randn(d.max_prompt, d.lm_d, generator=g, device=dev),
                   torch.randn(d.chunk, d.action, generator=g, device=dev))
    graph = fwd.capture()
    time_graph(graph)
    ms = sorted(time_graph(graph)[0] for _ in range(reps))[reps // 2]
    launches = sum(1 for l in fwd.schedule if l.kind != "torch")
    _log(f"[bench] pi05 forward: {ms:.3f} ms per chunk ({launches} HIP launches + {len(fwd.schedule) - launches} torch ops)")
    out = {"workload": "pi05: 3 views x SigLIP 27 layers, Gemma-2B prefix 18 layers x 816 rows, expert 10 steps x 18 "
                       "layers, chunk 50 (random weights, one HIP graph)", "ms_per_chunk": round(ms, 3),
           "launches": len(fwd.schedule),
           "reference_published_ms": {"value": 51.85, "hardware": "Jetson Thor", "source": "README.md:38"}}
    del fwd, graph
    torch.cuda.empty_cache()
    return out


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


def cpu_baseline(wl, max_rows=None, min_seconds=3.0):
    """The reference's CPU FP8 path (oracle/cpu_path.py: per-token quant,
    torch._scaled_mm via oneDNN, fp32 epilogue) over the config's calls, in its
    order, on a bounded sample: min(M, max_rows) tokens, fewer if one step of
    that would exceed ~min_seconds on this host (a 16-token step is timed
    first to decide). Whole steps are repeated until ~min_seconds of CPU time;
    with fewer than M tokens the time per step is extrapolated linearly to M
    (labelled). Value in the config's unit (GB/s for HBM-bound configs, TFLOP/s
    otherwise). A second line times the same step with dequantize-then-fp32-
    matmul (MKL), the oracle's formulation."""
    import torch
    from oracle import cpu_path
    M = wl.gemms[0].M
    gen = torch.Generator().manual_seed(0)
    weights = []
    for gm in wl.gemms:
        w8, sw = cpu_path.quant_rows(torch.randn((gm.N, gm.K), generator=gen) * 0.02)
        weights.append((gm, w8, sw, w8.float() * sw[:, None],
                        torch.randn(gm.N, generator=gen) * 0.01 if gm.bias else None,
                        torch.rand(gm.n_out, generator=gen).to(torch.bfloat16) if gm.gate else None))

    def inputs(r):
        return [(torch.randn((r, gm.K), generator=gen).to(torch.bfloat16),
                 torch.randn((r, gm.n_out), generator=gen).to(torch.bfloat16) if gm.residual else None)
                for gm, *_ in weights]

    def step(xs, fp32):
        for _ in range(wl.steps_per_unit):
            for (gm, w8, sw, wd, bias, gate), (x, res) in zip(weights, xs):
                q, sa = cpu_path.quant_rows(x)
                if fp32:
                    cpu_path.linear_fp32(q, sa, wd, bias=bias, act=gm.act, residual=res, gate=gate)
                else:
                    cpu_path.linear(q, sa, w8, sw, bias=bias, act=gm.act, residual=res, gate=gate)

    def timed(xs, fp32, budget):
        step(xs, fp32)  # warm-up (oneDNN primitive creation)
        n, t0 = 0, time.perf_counter()
        while True:
            step(xs, fp32)
            n += 1
            dt = time.perf_counter() - t0
            if dt >= budget or n >= 100000:
                return dt / n, n

    r = M if max_rows is None else min(M, max_rows)
    rc = min(r, 16)
    t_cal, _ = timed(inputs(rc), False, 0.0)
    if t_cal * r / rc > min_seconds:
        r = max(rc, int(min_seconds / t_cal * rc) // 16 * 16)
    xs = inputs(r)
    t8, n8 = timed(xs, False, min_seconds)
    t32, n32 = timed(xs, True, min_seconds / 2)
    t8, t32 = t8 * M / r, t32 * M / r

    def value(t):
        return round(wl.bytes / t / 1e9, 4) if wl.bound == "hbm" else round(wl.flops / t / 1e12, 6)

    unit = "GB/s" if wl.bound == "hbm" else "TFLOP/s"
    what = f"{n8} whole steps of {wl.key}" if r == M else \
        f"{n8} steps of {wl.key} on {r} of its {M} tokens, time extrapolated x{M / r:g} (linear in M)"
    return {"value": value(t8), "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "extrapolated": r != M, "seconds_per_step": round(t8, 6),
            "sample": f"{what}: per-token quant, torch._scaled_mm (oneDNN), fp32 epilogue on the host CPU "
                      "(reference GI decomposition)",
            "dequant_fp32_matmul": {"value": value(t32), "unit": unit, "seconds_per_step": round(t32, 6),
                                    "steps_timed": n32,
                                    "sample": "same calls and tokens: per-token quant, dequantize, fp32 matmul "
                                              "(MKL), fp32 epilogue"},
            "cpu": _cpu_model(), "os_cpu_count": os.cpu_count()}


CPU_ROWS = {"C1": None, "C2": None, "C3": 256, "C4": 256, "C5": 256}


def measure_sclk(wl, kernel_ms, wall_ms=20.0, launches=16):
    """Shader clock (MHz) while the dominant kernel runs back to back, and idle:
    ifx_sclk_probe on a second stream (default priority) spins `wall_ms` of the
    wall clock while at least 3x that much dominant-kernel work is queued ahead
    of it on the main stream."""
    import ctypes

    import torch
    from instinctflash_amd import _lib
    lib = _lib.load()
    khz = ctypes.c_int(0)
    _lib.check(lib.ifx_wall_clock_khz(ctypes.byref(khz)), "ifx_wall_clock_khz")
    ticks = int(wall_ms * khz.value)
    buf = torch.zeros(2, dtype=torch.int64, device="cuda")
    main, side = torch.cuda.Stream(), torch.cuda.Stream()
    main.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(main):  # eager first call on the capture stream (its workspace)
        wl.dominant_call(0)
    g = capture(lambda i: wl.dominant_call(i), launches, main)
    reps = max(1, int(3 * wall_ms / (kernel_ms * launches)) + 1)
    res = {}
    for busy in (True, False):
        torch.cuda.synchronize()
        if busy:
            for _ in range(reps):
                g.replay()  # on `main`, the capture stream
        _lib.check(lib.ifx_sclk_probe(buf.data_ptr(), ticks, side.cuda_stream), "ifx_sclk_probe")
        torch.cuda.synchronize()
        cyc, wt = (int(v) for v in buf.cpu())
        res["busy" if busy else "idle"] = round(cyc / (wt / (khz.value * 1e3)) / 1e6, 1)
    del g
    return {"sclk_mhz_under_kernel": res["busy"], "sclk_mhz_idle": res["idle"], "wall_clock_khz": khz.value,
            "method": f"ifx_sclk_probe ({wall_ms:g} ms of wall clock) on a second stream while "
                      f"{reps * launches} back-to-back launches of the dominant kernel run; idle: the probe alone"}


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
    ap.add_argument("--config", default="C5", choices=["C1", "C2", "C3", "C4", "C5"])
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

    results, metas = {}, {}
    order = [args.config] + ([] if args.no_others else [k for k in CONFIGS if k != args.config])
    for key in order:
        wl = CONFIGS[key](dev)
        steps = args.steps if key == args.config else max(10, min(args.steps, 20))
        _log(f"[bench] {key}: {wl.title} (pool {wl.pool}, {steps} steps)")
        m = measure(wl, steps, args.warmup)
        results[key] = summarize(wl, m)
        results[key]["steps"] = steps
        results[key]["roofline"] = roofline(wl, m)
        results[key]["calls"] = measure_calls(wl, 32 if wl.bound == "hbm" else 8)
        results[key]["hipblaslt"] = measure_vendor(wl, results[key]["calls"], 32 if wl.bound == "hbm" else 8)
        if key == args.config:
            head_m = m
            results[key]["roofline"].update(measure_sclk(wl, m["kernel_ms"]))
            sclk = results[key]["roofline"]["sclk_mhz_under_kernel"]
            if wl.bound == "mfma" and sclk > 0:
                # dense FP8 peak at the measured clock: 256 CUs x 8192 FLOP/clk
                at = 256 * 8192 * sclk * 1e6 / 1e12
                results[key]["roofline"]["peak_at_sclk"] = round(at, 1)
                results[key]["roofline"]["frac_at_sclk"] = round(results[key]["roofline"]["achieved"] / at, 4)
        wl.tensors, wl.ref = {}, {}  # keep the shapes (CPU baseline), free the device tensors
        metas[key] = wl
        del wl
        torch.cuda.empty_cache()

    wl, m, r = metas[args.config], head_m, results[args.config]
    value, unit = (r["gbs"], "GB/s") if wl.bound == "hbm" else (r["tflops"], "TFLOP/s")
    out = {
        "metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(m["step_ms"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8-e4m3 x fp8-e4m3 -> fp32 acc, bf16 out",
        "data": "synthetic (seeded torch.Generator on CPU, random-init weights quantized per channel)",
        "config": {"workload": f"{args.config}: {wl.title}", "M": wl.gemms[0].M, "gpu": arch,
                   "timed_unit": "4 flow-matching steps" if wl.steps_per_unit > 1 else "one pass"},
        "roofline": r["roofline"],
    }
    if not args.no_others:
        out["producers"] = measure_producers(dev)
        out["pi05_forward"] = measure_pi05(dev)
    if not args.no_cpu:
        for key in order:
            _log(f"[bench] CPU baseline {key} (reference CPU FP8 path)")
            results[key]["cpu_baseline"] = cpu_baseline(metas[key], CPU_ROWS[key])
        out["cpu_baseline"] = results[args.config]["cpu_baseline"]
    out["configs"] = results
    print(json.dumps(out))


if __name__ == "__main__":
    main()
