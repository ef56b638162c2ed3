"""Benchmark the HIP fused-group backend on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload resnet18] [--batch 32]

The default workload is the headline config: ResNet-18 fp32 at batch 32. One
step is one forward pass of the whole network over one batch of synthetic
N(0,1) images already resident in device memory (random-init weights of the
config's architecture and distributions). Other workloads (for the other
benchmark configs): ``mobilenetv2``, ``repvit_int8`` (bit-exact INT8 model),
``micro_gemm`` (the five fused GEMM+bias+ReLU shapes), ``int8_gemm``
(M = N = K = 4096, the compute-bound int8 shape).

Prints one JSON line: throughput, the dominant kernel's roofline (its
algorithmic work per launch over its average launch time, timed per launch
with HIP events on the library's stream), and the NumPy oracle timed on the
host cores over a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
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
CALIBRATION = "each Conv/Gemm LSUV-rescaled to unit output std as the reference exporters do"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----- CPU baseline: the oracle on a bounded sample -----------------------------

def cpu_baseline(graph, make_feeds, seconds: float = 12.0, what: str = "forwards") -> dict:
    """Time the NumPy oracle (a restatement of the reference executor) on
    single-image feeds, repeated until ``seconds`` have elapsed."""
    from oracle.reference import ReferenceExecutor

    ex = ReferenceExecutor(graph)
    feeds = make_feeds()
    ex.run(feeds)
    n, t0 = 0, time.perf_counter()
    while True:
        ex.run(feeds)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= 2:
            break
    return {"value": n / el, "unit": "images/s", "cores": 1, "kind": "port",
            "sample": f"{n} single-image {what} through the NumPy oracle (the reference "
                      f"executor's algorithm), {el:.1f} s, 1 thread, host of the GPU box"}


# ----- device timing -----------------------------------------------------------------

def time_module(c, feeds, steps: int, warmup: int, profile_iters: int, use_graph: bool = False):
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor

    ex = HipExecutor(c.module, use_graph=use_graph)
    try:
        ex._upload_feeds(feeds)
        ex.plan.run(warmup)
        ex.ctx.synchronize()
        ms = ex.plan.time_ms(0, steps)
        t1 = time.perf_counter()
        for _ in range(steps):
            ex.run(feeds)
        host_s = (time.perf_counter() - t1) / steps
        prof = ex.profile(profile_iters)
        arena = ex.arena_bytes
    finally:
        ex.close()
    return ms, host_s, prof, arena


def roofline(prof, *, traffic_json: str = "") -> tuple:
    per: dict = {}
    for launch, ms in prof:
        d = per.setdefault(launch.kernel_name, {"ms": 0.0, "flops": 0, "ops": 0, "bytes": 0,
                                                "launches": 0})
        d["ms"] += ms
        d["flops"] += launch.meta.get("flops", 0)
        d["ops"] += launch.meta.get("ops", 0)
        d["bytes"] += launch.meta.get("bytes", 0)
        d["launches"] += 1
    total = sum(d["ms"] for d in per.values())
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
    # The bound is the roofline's: matrix cores when the kernel's algorithmic
    # intensity (flops or ops per algorithmic HBM byte) is at or above the
    # ridge point peak/8 TB/s, else HBM bandwidth.
    work, peak, unit = ((d["flops"], PEAK_FP32_MFMA_TFLOPS, "TFLOP/s") if d["flops"] else
                        (d["ops"], PEAK_INT8_MFMA_TOPS, "TOP/s"))
    ridge = peak * 1e12 / (PEAK_HBM_GBS * 1e9)
    if work and (not d["bytes"] or work / d["bytes"] >= ridge):
        ach = work / d["launches"] / (avg * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": ach, "peak": peak, "unit": unit}
    else:
        ach = d["bytes"] / d["launches"] / (avg * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": ach, "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    if work and d["bytes"]:
        roof["intensity"] = work / d["bytes"]
    roof["frac"] = roof["achieved"] / roof["peak"]
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
    return roof, per


# ----- workloads ------------------------------------------------------------------------

def schedule_source(args):
    """The shipped measured schedules, or those of ``--schedules PATH`` (a
    tuner JSON cache), with shape-aware defaults for problems not in it."""
    if not args.schedules:
        return None
    from mdlc_amd.autotuner.tuner import AutotuneCache, Tuner

    return Tuner(AutotuneCache(args.schedules), tune_misses=False)


def network(args, name: str) -> dict:
    from mdlc_amd.compiler import compile_graph

    B = args.batch
    if name == "resnet18":
        from mdlc_amd.tools.build_resnet18 import build_resnet18 as build, make_input
    elif name == "mobilenetv2":
        from mdlc_amd.tools.build_mobilenetv2 import build_mobilenetv2 as build, make_input
    else:
        from mdlc_amd.tools.build_repvit_int8 import build_repvit_int8 as build, make_input
    x = make_input(B)
    t0 = time.perf_counter()
    folds = dict(fuse_residual=False, fuse_int8_epilogues=False) if args.no_fold else {}
    c = compile_graph(build(batch=B), feeds={"input": x}, conv_mode=args.conv_mode,
                      schedule_fn=schedule_source(args), **folds)
    log(f"{name} b={B}: compiled in {time.perf_counter() - t0:.1f} s, {len(c.module.plan)} launches")
    ms, host_s, prof, arena = time_module(c, {"input": x}, args.steps, args.warmup,
                                          args.profile_iters, args.graph)
    value = B * 1000.0 / ms
    log(f"{ms:.3f} ms/step, {value:.1f} images/s (arena {arena / 2**20:.1f} MiB)")
    traffic = TRAFFIC_JSON if (name == "resnet18" and B == 32 and not args.no_fold) else ""
    roof, _ = roofline(prof, traffic_json=traffic)
    int8 = name == "repvit_int8"
    work = sum(l.meta.get("ops" if int8 else "flops", 0) for l in c.module.plan)
    metric = METRIC if (name == "resnet18" and B == 32) else \
        f"{name} b={B} {'int8' if int8 else 'fp32'} images/sec"
    if int8:
        data = ("synthetic N(0,1) images, random-init int8 weights (w ~ N(0,0.05), per-channel "
                "scales), activation scales U(0.01,0.1)")
    else:
        data = ("synthetic N(0,1) images, random-init weights (Kaiming-normal conv/FC, BN gamma "
                "U(0.5,1.5) beta N(0,0.1) mean N(0,0.1) var U(0.5,1.5); " + CALIBRATION + ")")
    line = {
        "metric": metric, "value": value, "unit": "images/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "i8" if int8 else "f32", "data": data,
        "config": {"workload": f"{name}_{'int8' if int8 else 'fp32'}_b{B}", "batch": B,
                   "image": [3, 224, 224], "conv_mode": args.conv_mode,
                   "backend_folds": not args.no_fold,
                   "launches": len(c.module.plan), "gop_per_step": work / 1e9,
                   ("network_tops" if int8 else "network_tflops"): work / (ms * 1e-3) / 1e12,
                   "host_buffer_images_per_s": B / host_s},
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        c1 = compile_graph(build(batch=1), feeds={"input": make_input(1, seed=7)})
        line["cpu_baseline"] = cpu_baseline(c1.graph, lambda: {"input": make_input(1, seed=7)},
                                            what=f"{name} forwards")
    return line


def micro_gemm(args) -> dict:
    from mdlc_amd.compiler import compile_graph
    from mdlc_amd.tools.micro_gemm import SHAPES, build_micro_gemm

    shapes, total_flops, total_ms, cpu = {}, 0.0, 0.0, {}
    for M, N, K in SHAPES:
        g, feeds = build_micro_gemm(M, N, K)
        c = compile_graph(g, feeds=feeds, schedule_fn=schedule_source(args))
        ms, _, _, _ = time_module(c, feeds, args.steps * 10, args.warmup, args.profile_iters)
        fl = 2.0 * M * N * K
        key = f"{M}x{N}x{K}"
        shapes[key] = {"us": ms * 1e3, "tflops": fl / (ms * 1e-3) / 1e12,
                       "frac_fp32_peak": fl / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS,
                       "launches": len(c.module.plan)}
        total_flops += fl
        total_ms += ms
        if not args.no_cpu_baseline:
            from oracle.reference import run_reference

            run_reference(c.graph, feeds)
            t0, n = time.perf_counter(), 0
            while time.perf_counter() - t0 < 1.5 or n < 2:
                run_reference(c.graph, feeds)
                n += 1
            cpu[key] = fl * n / (time.perf_counter() - t0) / 1e9
        log(f"{key}: {ms * 1e3:.1f} us, {shapes[key]['tflops']:.1f} TFLOP/s")
    line = {"metric": "fused GEMM+bias+ReLU micro-workload TFLOP/s (5 ResNet-18 batch-1 shapes)",
            "value": total_flops / (total_ms * 1e-3) / 1e12, "unit": "TFLOP/s", "n_gpus": 1,
            "steps": args.steps * 10, "warmup": args.warmup, "ms_per_step": total_ms,
            "higher_is_better": True, "scaling": "strong", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic A, B, bias ~ N(0,1)/sqrt(K), fixed seed per shape",
            "config": {"workload": "micro_gemm_bias_relu", "shapes": shapes}}
    if cpu:
        line["cpu_baseline"] = {
            "value": sum(cpu.values()) / len(cpu), "unit": "GFLOP/s (mean over shapes)",
            "cores": 1, "kind": "port",
            "sample": "each shape through the NumPy oracle (A @ B + bias, relu) for >= 1.5 s: "
                      + ", ".join(f"{k}: {v:.1f}" for k, v in cpu.items())}
    return line


def int8_gemm(args) -> dict:
    import numpy as np

    from mdlc_amd.compiler import compile_graph
    from mdlc_amd.tools.graph_builder import GraphBuilder

    M = N = K = args.size
    rng = np.random.default_rng(0)
    b = GraphBuilder("i8gemm")
    b.input("xq", (M, K), dtype="int8")
    b.const("w", rng.integers(-127, 128, (N, K)).astype(np.int8))
    b.const("b", rng.integers(-1000, 1000, N).astype(np.int32))
    b.const("m", rng.uniform(2e-6, 1e-5, N).astype(np.float32))
    b.node("QGemm", ["xq", "w", "b", "m"], "y", transB=1)
    b.output("y")
    feeds = {"xq": rng.integers(-127, 128, (M, K)).astype(np.int8)}
    c = compile_graph(b.graph(), feeds=feeds, schedule_fn=schedule_source(args))
    ms, _, prof, _ = time_module(c, feeds, args.steps, args.warmup, args.profile_iters)
    tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    roof, _ = roofline(prof)
    log(f"int8 GEMM {M}^3: {ms * 1e3:.1f} us, {tops:.0f} TOP/s")
    return {"metric": f"int8 GEMM {M}x{N}x{K} TOP/s (int32 acc, requantized int8 out)",
            "value": tops, "unit": "TOP/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True,
            "scaling": "strong", "vs_baseline": None, "dtype": "i8", "data": "synthetic int8 codes",
            "config": {"workload": "int8_gemm", "M": M, "N": N, "K": K}, "roofline": roof}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="resnet18",
                    choices=["resnet18", "mobilenetv2", "repvit_int8", "micro_gemm", "int8_gemm"])
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--size", type=int, default=4096, help="int8_gemm M = N = K")
    ap.add_argument("--conv-mode", default="implicit", choices=["implicit", "im2col"])
    ap.add_argument("--schedules", default="", help="tuner JSON cache to use instead of the "
                    "shipped mdlc_amd/autotuner/tuned_gfx950.json")
    ap.add_argument("--graph", action="store_true", help="replay the plan as a hipGraph")
    ap.add_argument("--no-fold", action="store_true",
                    help="the reference's fused groups only (no residual / int8 / pool folds)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-iters", type=int, default=3)
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "inference shards by batch across GPUs, which is not part of this build",
              file=sys.stderr)
        return 2
    if args.workload == "micro_gemm":
        line = micro_gemm(args)
    elif args.workload == "int8_gemm":
        line = int8_gemm(args)
    else:
        line = network(args, args.workload)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
