"""Benchmark the HIP fused-group backend on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload resnet18] [--batch 32]

The default workload is the headline config: ResNet-18 fp32 at batch 32. One
step is one forward pass of the whole network over one batch of synthetic
N(0,1) images already resident in device memory (random-init weights of the
config's architecture and distributions). The default run also measures the
other benchmark configs and reports them under ``config.secondary``:
ResNet-18 b=1, MobileNetV2 b=1 and b=32, the RepViT-style INT8 model at b=32,
the five fused GEMM+bias+ReLU micro shapes and the int8 GEMM at 4096^3
(``--no-secondary`` skips them). Each config can also be run on its own with
``--workload`` (``mobilenetv2``, ``repvit_int8``, ``micro_gemm``,
``int8_gemm``).

Each workload's plan first runs untimed for ``--settle-ms`` of device time
(100 ms by default; ``settle_ms`` in the line), then ``--warmup`` untimed
steps, then exactly ``--steps`` timed ones: from an idle device the GPU clock
needs tens of milliseconds of load to reach its sustained value, and a few
warm-up steps of a sub-millisecond forward end well before that.

Prints one JSON line: throughput; the dominant kernel's roofline (its
algorithmic work per launch over its average launch time, timed per launch
with HIP events on the library's stream), also for the kernel together with
the split-K reduce or stream-K fix-up launch that finishes its output; and
the NumPy oracle timed on the host cores over a bounded sample, before the
first device call.
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
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "ResNet-18 b=32 fp32 images/sec; fused GEMM/conv TFLOP/s & % MFMA peak"
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "resnet18_b32_traffic.json")
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_INT8_MFMA_TOPS = 5000.0
PEAK_HBM_GBS = 8000.0
FINISHERS = ("splitk_reduce", "streamk_fixup")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----- host description and the CPU baseline ---------------------------------------

def host_info() -> dict:
    """What the CPU baseline ran on: model, logical CPUs, the CPUs this
    process may use, thread settings and the BLAS thread pool."""
    import numpy  # noqa: F401  (loads the bundled BLAS so it can be inspected)

    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    pools = []
    try:
        from threadpoolctl import threadpool_info

        pools = [{"api": p.get("internal_api"), "threads": p.get("num_threads")}
                 for p in threadpool_info()]
    except Exception:
        pass
    env = {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS",
                                          "MKL_NUM_THREADS")}
    return {"cpu_model": model, "cpu_count": os.cpu_count(), "usable_cpus": usable,
            "env": env, "blas_pools": pools}


def _threads_used(info: dict) -> int:
    """Threads the oracle can run on: its convolutions are single-threaded
    NumPy einsum loops, its matrix products use the BLAS pool."""
    return max([1] + [p["threads"] or 1 for p in info["blas_pools"]])


def cpu_network(name: str, batch: int, *, seconds: float = 0.0, sample: int = 0) -> dict:
    """The NumPy oracle (a restatement of the reference executor) on the
    host for one network workload: at batch 1, single-image forwards
    repeated for ``seconds``; at a larger batch, one forward over ``sample``
    of the batch's images (the whole batch when ``sample`` equals it)."""
    from mdlc_amd.compiler import compile_graph
    from oracle.reference import ReferenceExecutor

    build, make_input = builders(name)
    info = host_info()
    threads = _threads_used(info)
    how = ("einsum convolutions, single-threaded; BLAS matrix products on up to "
           f"{threads} threads" if name != "repvit_int8" else
           "exact int64 NumPy products with the requantization, single-threaded")
    if batch == 1:
        x = make_input(1, seed=7)
        ex = ReferenceExecutor(compile_graph(build(batch=1), feeds={"input": x}).graph)
        ex.run({"input": x})
        n, t0 = 0, time.perf_counter()
        while True:
            ex.run({"input": x})
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds and n >= 2:
                break
        value, what = n / el, f"{n} single-image forwards ({el:.1f} s)"
    else:
        k = min(sample or batch, batch)
        x = make_input(batch)[:k]
        ex = ReferenceExecutor(compile_graph(build(batch=k), feeds={"input": x}).graph)
        t0 = time.perf_counter()
        ex.run({"input": x})
        el = time.perf_counter() - t0
        value = k / el
        what = (f"one batch-{batch} forward ({el:.1f} s)" if k == batch else
                f"one forward over {k} of the batch's {batch} images ({el:.1f} s; per-image "
                f"work is independent of the batch)")
    log(f"cpu {name} b={batch}: {value:.2f} images/s")
    return {"value": value, "unit": "images/s", "cores": threads, "kind": "port",
            "sample": f"{what} of {name} through the NumPy oracle (the reference executor's "
                      f"algorithm: {how}), host of the GPU box",
            "host": info}


def cpu_micro(compiled) -> dict:
    """Each micro GEMM through the oracle (A @ B + bias, relu; BLAS) for
    at least a second."""
    from oracle.reference import run_reference

    rates = {}
    for (M, N, K), c, feeds in compiled:
        run_reference(c.graph, feeds)
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < 1.0 or n < 2:
            run_reference(c.graph, feeds)
            n += 1
        rates[f"{M}x{N}x{K}"] = 2.0 * M * N * K * n / (time.perf_counter() - t0) / 1e9
    info = host_info()
    log("cpu micro GEMMs: " + ", ".join(f"{k} {v:.1f} GFLOP/s" for k, v in rates.items()))
    return {"value": sum(rates.values()) / len(rates), "unit": "GFLOP/s (mean over shapes)",
            "cores": _threads_used(info), "kind": "port", "host": info,
            "sample": "each shape through the NumPy oracle (A @ B + bias, relu; BLAS) for >= 1 s: "
                      + ", ".join(f"{k}: {v:.1f}" for k, v in rates.items())}


def cpu_int8(feeds, w, size: int) -> dict:
    """32 rows of the int8 GEMM through the oracle's exact int64 product and
    requantization."""
    import numpy as np

    from oracle.quant import gemm_acc, requant

    rows = 32
    t0 = time.perf_counter()
    requant(gemm_acc(feeds["xq"][:rows], w, None), np.ones(size, np.float32) * 1e-5)
    el = time.perf_counter() - t0
    log(f"cpu int8 GEMM: {2.0 * rows * size * size / el / 1e9:.1f} GOP/s")
    return {"value": 2.0 * rows * size * size / el / 1e12, "unit": "TOP/s", "cores": 1, "kind": "port",
            "host": host_info(),
            "sample": f"{rows} of the {size} rows through the oracle's exact int64 matmul + requant "
                      f"({el:.2f} s; NumPy integer matmul, one thread)"}


# ----- device timing ------------------------------------------------------------------

SETTLE_MS = 100.0          # device time run before each workload's warm-up (--settle-ms)
SETTLE_MAX_STEPS = 20000


def settle(ex, settle_ms: float) -> int:
    """Run the plan for about ``settle_ms`` of device time, untimed, so the
    GPU is at its sustained clock when the warm-up and timed steps start: from
    an idle device the clock takes tens of milliseconds of load to settle
    (ResNet-18 b=32 measured 0.909-0.914 ms a forward after 5 warm-up steps,
    0.893 ms after 100 or 300; int8 4096^3 74 us against 66 us). Returns the
    number of plan runs."""
    if settle_ms <= 0:
        return 0
    per = ex.plan.time_ms(0, 2)                 # ms of one run, measured on the device
    n = int(min(SETTLE_MAX_STEPS, max(1, math.ceil(settle_ms / max(per, 1e-3)))))
    ex.plan.run(n)
    ex.ctx.synchronize()
    return n


def time_module(c, feeds, steps: int, warmup: int, profile_iters: int, use_graph: bool = False,
                host_loop: bool = True):
    """(ms per step by events, host seconds per step including the feed
    upload and output read, per-launch profile, arena bytes). The plan first
    runs for SETTLE_MS of device time (``settle``), then ``warmup`` untimed
    steps, then exactly ``steps`` timed ones."""
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor

    ex = HipExecutor(c.module, use_graph=use_graph)
    try:
        ex._upload_feeds(feeds)
        settle(ex, SETTLE_MS)
        ex.plan.run(warmup)
        ex.ctx.synchronize()
        ms = ex.plan.time_ms(0, steps)
        host_s = None
        if host_loop:
            t1 = time.perf_counter()
            for _ in range(steps):
                ex.run(feeds)
            host_s = (time.perf_counter() - t1) / steps
        prof = ex.profile(profile_iters)
        arena = ex.arena_bytes
    finally:
        ex.close()
    return ms, host_s, prof, arena


def _bound(work: float, nbytes: float, peak: float) -> bool:
    """MFMA-bound when the algorithmic intensity reaches the ridge point
    peak / HBM bandwidth."""
    ridge = peak * 1e12 / (PEAK_HBM_GBS * 1e9)
    return bool(work) and (not nbytes or work / nbytes >= ridge)


def _rate(work: float, nbytes: float, ms: float, int8: bool) -> dict:
    peak = PEAK_INT8_MFMA_TOPS if int8 else PEAK_FP32_MFMA_TFLOPS
    if _bound(work, nbytes, peak):
        ach = work / (ms * 1e-3) / 1e12
        r = {"bound": "mfma", "achieved": ach, "peak": peak, "unit": "TOP/s" if int8 else "TFLOP/s"}
    else:
        ach = nbytes / (ms * 1e-3) / 1e9
        r = {"bound": "hbm", "achieved": ach, "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    r["frac"] = r["achieved"] / r["peak"]
    return r


def roofline(prof, *, traffic_json: str = "", verbose: bool = True, step_ms: float = None) -> tuple:
    """Roofline of the kernel with the largest share of the step, per launch,
    plus the same kernel together with the split-K reduce / stream-K fix-up
    launches that finish its output (``group``). Where a step is that one
    launch (``step_ms`` given), its duration is the timed region's: events
    attached to each dispatch of a one-launch plan read several us long
    against the back-to-back launches (81 against 72.6 us at int8 4096^3)."""
    per: dict = {}
    for launch, ms in prof:
        d = per.setdefault(launch.kernel_name, {"ms": 0.0, "flops": 0, "ops": 0, "bytes": 0,
                                                "launches": 0, "direct_flops": 0})
        d["ms"] += ms
        d["flops"] += launch.meta.get("flops", 0)
        d["direct_flops"] += launch.meta.get("direct_flops", 0)
        d["ops"] += launch.meta.get("ops", 0)
        d["bytes"] += launch.meta.get("bytes", 0)
        d["launches"] += 1
    total = sum(d["ms"] for d in per.values())
    if verbose:
        for name, d in sorted(per.items(), key=lambda kv: -kv[1]["ms"])[:24]:
            if d["flops"]:
                rate = f"{d['flops'] / d['ms'] / 1e9:8.1f} TFLOP/s"
            elif d["ops"]:
                rate = f"{d['ops'] / d['ms'] / 1e9:8.1f} TOP/s"
            else:
                rate = f"{d['bytes'] / d['ms'] / 1e6:8.1f} GB/s"
            log(f"  {name:58s} {d['launches']:3d}x {d['ms']:8.3f} ms {rate}")
    name, d = max(per.items(), key=lambda kv: kv[1]["ms"])
    avg = d["ms"] / d["launches"]
    dispatch_ms = None
    if step_ms is not None and len(per) == 1 and d["launches"] == 1:
        dispatch_ms, avg = avg, step_ms
    int8 = not d["flops"] and bool(d["ops"])
    work = d["flops"] or d["ops"]
    roof = _rate(work / d["launches"], d["bytes"] / d["launches"], avg, int8)
    if work and d["bytes"]:
        roof["intensity"] = work / d["bytes"]
    roof["traffic"] = None
    if traffic_json and os.path.exists(traffic_json):
        # HBM bytes per dispatch from the committed rocprofv3 FETCH_SIZE /
        # WRITE_SIZE runs of this workload (copy-calibrated); valid only for
        # the kernel those runs measured.
        with open(traffic_json) as f:
            m = json.load(f)["kernels"].get(name)
        if m:
            roof["traffic"] = m["traffic_bytes"]
    roof.update({"kernel": name, "launches_per_step": d["launches"], "avg_launch_ms": avg,
                 "share_of_step": d["ms"] / total})
    if dispatch_ms is not None:
        roof["avg_launch_from"] = "timed region (one launch a step)"
        roof["dispatch_event_ms"] = dispatch_ms
    if d["direct_flops"]:
        # a Winograd convolution: "achieved" counts the multiply-adds it
        # performs (16 per 2x2 tile and channel pair); the direct
        # convolution's count over the same time is reported beside it
        roof["algorithm"] = "winograd F(2x2,3x3)"
        roof["direct_conv_equivalent"] = d["direct_flops"] / d["launches"] / (avg * 1e-3) / 1e12
    # the launches that finish this kernel's output (same graph node, next in the plan)
    group_ms, finishers = [], set()
    for i, (launch, ms) in enumerate(prof):
        if launch.kernel_name != name:
            continue
        t = ms
        for nxt, nms in prof[i + 1:]:
            if nxt.kind in FINISHERS and nxt.meta.get("node") is launch.meta.get("node"):
                t += nms
                finishers.add(nxt.kernel_name)
            else:
                break
        group_ms.append(t)
    if finishers:
        gavg = sum(group_ms) / len(group_ms)
        g = _rate(work / d["launches"], d["bytes"] / d["launches"], gavg, int8)
        roof["group"] = {"kernels": [name] + sorted(finishers), "avg_ms": gavg,
                         "achieved": g["achieved"], "frac": g["frac"]}
    return roof, per


# ----- workloads ------------------------------------------------------------------------

def builders(name: str):
    if name == "resnet18":
        from mdlc_amd.tools.build_resnet18 import build_resnet18 as build, make_input
    elif name == "mobilenetv2":
        from mdlc_amd.tools.build_mobilenetv2 import build_mobilenetv2 as build, make_input
    else:
        from mdlc_amd.tools.build_repvit_int8 import build_repvit_int8 as build, make_input
    return build, make_input


def schedule_source(args):
    """The shipped measured schedules, or those of ``--schedules PATH`` (a
    tuner JSON cache), with shape-aware defaults for problems not in it."""
    if not args.schedules:
        return None
    from mdlc_amd.autotuner.tuner import AutotuneCache, Tuner

    return Tuner(AutotuneCache(args.schedules), tune_misses=False)


def compile_network(args, name: str, batch: int):
    from mdlc_amd.compiler import compile_graph

    build, make_input = builders(name)
    x = make_input(batch)
    t0 = time.perf_counter()
    folds = dict(fuse_residual=False, fuse_int8_epilogues=False) if args.no_fold else {}
    c = compile_graph(build(batch=batch), feeds={"input": x}, conv_mode=args.conv_mode,
                      schedule_fn=schedule_source(args),
                      winograd={"auto": "auto", "always": True, "never": False}[args.winograd], **folds)
    log(f"{name} b={batch}: compiled in {time.perf_counter() - t0:.1f} s, {len(c.module.plan)} launches")
    return c, {"input": x}


def network(args, name: str, batch: int, *, steps: int, headline: bool) -> dict:
    c, feeds = compile_network(args, name, batch)
    cold = cold_compile_seconds(c) if headline else None
    ms, host_s, prof, arena = time_module(c, feeds, steps, args.warmup, args.profile_iters,
                                          args.graph, host_loop=headline)
    value = batch * 1000.0 / ms
    log(f"{name} b={batch}: {ms:.3f} ms/step, {value:.1f} images/s (arena {arena / 2**20:.1f} MiB)")
    traffic = TRAFFIC_JSON if (name == "resnet18" and batch == 32 and not args.no_fold) else ""
    roof, _ = roofline(prof, traffic_json=traffic, verbose=headline)
    int8 = name == "repvit_int8"
    key = "ops" if int8 else "flops"
    # executed: the multiply-adds the kernels perform (a Winograd conv performs
    # fewer than the convolution it computes); algorithmic: 2*M*N*K of every
    # conv/GEMM as the reference's im2col formulation counts it
    executed = sum(l.meta.get(key, 0) for l in c.module.plan)
    algorithmic = sum(l.meta.get("direct_flops", l.meta.get(key, 0)) for l in c.module.plan)
    metric = METRIC if (name == "resnet18" and batch == 32) else \
        f"{name} b={batch} {'int8' if int8 else 'fp32'} images/sec"
    g, r = ("gop", "tops") if int8 else ("gflop", "tflops")
    line = {"metric": metric, "value": value, "unit": "images/s", "ms_per_step": ms,
            "steps": steps, "dtype": "i8" if int8 else "f32", "workload": workload_key(name, batch),
            "launches": len(c.module.plan),
            f"algorithmic_{g}_per_step": algorithmic / 1e9,
            f"network_{r}": algorithmic / (ms * 1e-3) / 1e12,
            f"executed_{g}_per_step": executed / 1e9,
            f"executed_{r}": executed / (ms * 1e-3) / 1e12,
            "roofline": roof}
    if host_s:
        line["host_buffer_images_per_s"] = batch / host_s
    if cold is not None:
        line["cold_compile_s"] = cold
        log(f"{name} b={batch}: cold hipRTC compile {cold:.1f} s")
    return line


def micro_compiled(args) -> list:
    from mdlc_amd.compiler import compile_graph
    from mdlc_amd.tools.micro_gemm import SHAPES, build_micro_gemm

    out = []
    for M, N, K in SHAPES:
        g, feeds = build_micro_gemm(M, N, K)
        out.append(((M, N, K), compile_graph(g, feeds=feeds, schedule_fn=schedule_source(args)), feeds))
    return out


def micro_gemm(args, *, steps: int, cpu: bool) -> dict:
    shapes, total_flops, total_ms = {}, 0.0, 0.0
    compiled = micro_compiled(args)
    cpu_line = cpu_micro(compiled) if cpu else None      # host leg first, before any device call
    for (M, N, K), c, feeds in compiled:
        ms, _, prof, _ = time_module(c, feeds, steps, args.warmup, args.profile_iters,
                                     host_loop=False)
        fl = 2.0 * M * N * K
        key = f"{M}x{N}x{K}"
        roof, _ = roofline(prof, verbose=False, step_ms=ms if len(c.module.plan) == 1 else None)
        shapes[key] = {"us": ms * 1e3, "tflops": fl / (ms * 1e-3) / 1e12,
                       "frac_fp32_peak": fl / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS,
                       "launches": len(c.module.plan),
                       "step_roofline": _rate(fl, 4.0 * (M * K + K * N + N + M * N), ms, False),
                       "roofline": roof}
        total_flops += fl
        total_ms += ms
        log(f"micro {key}: {ms * 1e3:.1f} us, {shapes[key]['tflops']:.1f} TFLOP/s "
            f"({len(c.module.plan)} launches)")
    line = {"metric": "fused GEMM+bias+ReLU micro-workload TFLOP/s (5 ResNet-18 batch-1 shapes)",
            "value": total_flops / (total_ms * 1e-3) / 1e12, "unit": "TFLOP/s",
            "ms_per_step": total_ms, "steps": steps, "dtype": "f32",
            "workload": "micro_gemm_bias_relu", "shapes": shapes}
    if cpu_line:
        line["cpu_baseline"] = cpu_line
    return line


def int8_problem(size: int):
    """(feeds, weights, graph) of the requantized int8 GEMM at M = N = K = size."""
    import numpy as np

    from mdlc_amd.tools.graph_builder import GraphBuilder

    rng = np.random.default_rng(0)
    b = GraphBuilder("i8gemm")
    b.input("xq", (size, size), dtype="int8")
    w = rng.integers(-127, 128, (size, size)).astype(np.int8)
    b.const("w", w)
    b.const("b", rng.integers(-1000, 1000, size).astype(np.int32))
    b.const("m", rng.uniform(2e-6, 1e-5, size).astype(np.float32))
    b.node("QGemm", ["xq", "w", "b", "m"], "y", transB=1)
    b.output("y")
    return {"xq": rng.integers(-127, 128, (size, size)).astype(np.int8)}, w, b.graph()


def int8_gemm(args, *, steps: int, cpu: bool) -> dict:
    from mdlc_amd.compiler import compile_graph

    M = N = K = args.size
    feeds, w, g = int8_problem(M)
    c = compile_graph(g, feeds=feeds, schedule_fn=schedule_source(args))
    cpu_line = cpu_int8(feeds, w, M) if cpu else None   # host leg first
    ms, _, prof, _ = time_module(c, feeds, steps, args.warmup, args.profile_iters, host_loop=False)
    tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    roof, _ = roofline(prof, verbose=False, step_ms=ms)
    log(f"int8 GEMM {M}^3: {ms * 1e3:.1f} us, {tops:.0f} TOP/s")
    line = {"metric": f"int8 GEMM {M}x{N}x{K} TOP/s (int32 acc, requantized int8 out)",
            "value": tops, "unit": "TOP/s", "ms_per_step": ms, "steps": steps, "dtype": "i8",
            "workload": "int8_gemm", "M": M, "N": N, "K": K, "roofline": roof}
    if cpu_line:
        line["cpu_baseline"] = cpu_line
    return line


def full_line(args, part: dict, *, scaling: str, data: str, config: dict) -> dict:
    """The driver's JSON contract around one measured part."""
    keep = {k: v for k, v in part.items()
            if k in ("launches", "host_buffer_images_per_s", "cold_compile_s", "shapes", "M", "N", "K")
            or k.startswith(("algorithmic_", "executed_", "network_"))}
    out = {"metric": part["metric"], "value": part["value"], "unit": part["unit"], "n_gpus": 1,
           "steps": part["steps"], "warmup": args.warmup, "settle_ms": SETTLE_MS,
           "ms_per_step": part["ms_per_step"],
           "higher_is_better": True, "scaling": scaling, "vs_baseline": None,
           "dtype": part["dtype"], "data": data,
           "config": {"workload": part["workload"], **config, **keep}}
    if "roofline" in part:
        out["roofline"] = part["roofline"]
    if "cpu_baseline" in part:
        out["cpu_baseline"] = part["cpu_baseline"]
    return out


def data_text(name: str) -> str:
    if name == "repvit_int8":
        return ("synthetic N(0,1) images, random-init int8 weights (w ~ N(0,0.05), per-channel "
                "scales), activation scales U(0.01,0.1)")
    if name in ("micro_gemm", "int8_gemm"):
        return ("synthetic A, B, bias ~ N(0,1)/sqrt(K), fixed seed per shape" if name == "micro_gemm"
                else "synthetic int8 codes")
    init = ("synthetic N(0,1) images, random-init weights (Kaiming-normal conv/FC, BN gamma "
            "U(0.5,1.5) beta N(0,0.1) mean N(0,0.1) var U(0.5,1.5)")
    if name == "resnet18":
        return init + ", used as drawn like the reference's ResNet-18 exporter)"
    return init + "; each Conv/Gemm LSUV-rescaled to unit output std, as the reference's " \
        "MobileNetV2 exporter does)"


SECONDARY = (("resnet18", 1, 50), ("mobilenetv2", 1, 50), ("mobilenetv2", 32, 20),
             ("repvit_int8", 32, 20))


def workload_key(name: str, batch: int) -> str:
    return f"{name}_{'int8' if name == 'repvit_int8' else 'fp32'}_b{batch}"


def cpu_legs(args, headline: str, batch: int, with_secondary: bool) -> dict:
    """Every CPU baseline of the run, timed before the first device call:
    the headline workload's, then each secondary config's on a bounded
    sample (about 45 s in all)."""
    out = {workload_key(headline, batch): cpu_network(headline, batch, seconds=6.0, sample=batch)}
    if with_secondary:
        for name, b, _ in SECONDARY:
            key = workload_key(name, b)
            if key not in out:
                out[key] = (cpu_network(name, 1, seconds=4.0) if b == 1 else
                            cpu_network(name, b, sample=8 if name == "mobilenetv2" else 4))
        out["micro_gemm_bias_relu"] = cpu_micro(micro_compiled(args))
        feeds, w, _ = int8_problem(4096)
        out["int8_gemm_4096"] = cpu_int8(feeds, w, 4096)
    return out


def secondary(args, cpu: dict) -> dict:
    """The other benchmark configs, each with its own roofline block and the
    CPU baseline measured for it before the first device call."""
    out = {}
    for name, batch, steps in SECONDARY:
        part = network(args, name, batch, steps=steps, headline=False)
        if part["workload"] in cpu:
            part["cpu_baseline"] = cpu[part["workload"]]
        out[part["workload"]] = {k: v for k, v in part.items() if k not in ("workload", "dtype")}
    out["micro_gemm_bias_relu"] = micro_gemm(args, steps=200, cpu=False)
    if "micro_gemm_bias_relu" in cpu:
        out["micro_gemm_bias_relu"]["cpu_baseline"] = cpu["micro_gemm_bias_relu"]
    size = args.size
    args.size = 4096
    out["int8_gemm_4096"] = int8_gemm(args, steps=20, cpu=False)
    if "int8_gemm_4096" in cpu:
        out["int8_gemm_4096"]["cpu_baseline"] = cpu["int8_gemm_4096"]
    args.size = size
    return out


def cold_compile_seconds(c) -> float:
    """hipRTC compile time of the module with no code-object cache."""
    from mdlc_amd.codegen.hip.hiprtc_runtime import compile_code_object

    t0 = time.perf_counter()
    compile_code_object(c.module.sources(), use_cache=False)
    return time.perf_counter() - t0


def main(argv=None) -> int:
    global SETTLE_MS
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="resnet18",
                    choices=["resnet18", "mobilenetv2", "repvit_int8", "micro_gemm", "int8_gemm"])
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--size", type=int, default=4096, help="int8_gemm M = N = K")
    ap.add_argument("--conv-mode", default="implicit", choices=["implicit", "im2col"])
    ap.add_argument("--winograd", default="auto", choices=["auto", "always", "never"],
                    help="3x3 stride-1 convs as Winograd F(2x2, 3x3): where its grid fills half "
                         "the CUs (auto), always, or never (the implicit GEMM)")
    ap.add_argument("--schedules", default="", help="tuner JSON cache to use instead of the "
                    "shipped mdlc_amd/autotuner/tuned_gfx950.json")
    ap.add_argument("--graph", action="store_true", help="replay the plan as a hipGraph")
    ap.add_argument("--no-fold", action="store_true",
                    help="the reference's fused groups only (no residual / int8 / pool folds)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="measure only the selected workload")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="device time each workload's plan runs, untimed, before its warm-up "
                         "steps, so the GPU is at its sustained clock (0: none)")
    ap.add_argument("--profile-iters", type=int, default=25,
                    help="runs of the plan whose per-launch median the roofline uses")
    args = ap.parse_args(argv)
    SETTLE_MS = args.settle_ms
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "inference shards by batch across GPUs, which is not part of this build",
              file=sys.stderr)
        return 2
    cpu = not args.no_cpu_baseline
    w = args.workload
    if w == "micro_gemm":
        part = micro_gemm(args, steps=args.steps * 10, cpu=cpu)
        line = full_line(args, part, scaling="strong", data=data_text(w), config={})
    elif w == "int8_gemm":
        part = int8_gemm(args, steps=args.steps, cpu=cpu)
        line = full_line(args, part, scaling="strong", data=data_text(w), config={})
    else:
        with_sec = w == "resnet18" and args.batch == 32 and not args.no_secondary
        cpu_lines = cpu_legs(args, w, args.batch, with_sec) if cpu else {}
        part = network(args, w, args.batch, steps=args.steps, headline=True)
        if part["workload"] in cpu_lines:
            part["cpu_baseline"] = cpu_lines[part["workload"]]
        line = full_line(args, part, scaling="weak", data=data_text(w),
                         config={"batch": args.batch, "image": [3, 224, 224],
                                 "conv_mode": args.conv_mode, "winograd": args.winograd,
                                 "backend_folds": not args.no_fold})
        if with_sec:
            line["config"]["secondary"] = secondary(args, cpu_lines)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
