"""Tune the MFMA schedules of every GEMM/conv problem in a model.

    python -m mdlc_amd.tools.tune --model resnet18 --batch 32 --precompile   # CPU: fill the code-object cache
    python -m mdlc_amd.tools.tune --model resnet18 --batch 32                # device: measure, write JSON

The first form needs no GPU: hipRTC compiles every candidate module into the
on-disk code-object cache, so the measuring run on the device spends its
time timing rather than compiling. Results merge into
``mdlc_amd/autotuner/tuned_gfx950.json`` (or ``--out``).
"""

from __future__ import annotations

import argparse
import sys
import time
from concurrent.futures import ProcessPoolExecutor

from mdlc_amd.autotuner.tuner import (
    TUNED_PATH, AutotuneCache, is_int8, precompile, problem_candidates, problem_key, tune_problem,
)
from mdlc_amd.codegen.schedule import default_qdw_schedule, default_qschedule, default_schedule


class _Recorder:
    def __init__(self) -> None:
        self.problems: dict = {}

    def schedule_problem(self, problem: dict):
        self.problems.setdefault(problem_key(problem), dict(problem))
        return default_schedule(problem["M"], problem["N"], problem["K"])

    def __call__(self, node, mnk):
        return default_schedule(*mnk)


def model_problems(model: str, batch: int, conv_mode: str) -> list:
    from mdlc_amd.compiler import compile_graph

    if model == "int8_gemm":          # the square int8 GEMM benchmark, M = N = K = batch
        return [{"kind": "qgemm", "M": batch, "N": batch, "K": batch, "out_f32": False}]
    if model == "fp32_gemm":          # a square dense fp32 GEMM, M = N = K = batch
        return [{"kind": "gemm", "M": batch, "N": batch, "K": batch}]
    if model == "micro":              # the five fused GEMM+bias+ReLU micro shapes
        from mdlc_amd.tools.micro_gemm import SHAPES
        return [{"kind": "gemm", "M": M, "N": N, "K": K} for M, N, K in SHAPES]
    if model == "resnet18":
        from mdlc_amd.tools.build_resnet18 import build_resnet18
        graph = build_resnet18(batch=batch, calibrate=False)
    elif model == "mobilenetv2":
        from mdlc_amd.tools.build_mobilenetv2 import build_mobilenetv2
        graph = build_mobilenetv2(batch=batch, calibrate=False)
    elif model == "repvit_int8":
        from mdlc_amd.tools.build_repvit_int8 import build_repvit_int8
        graph = build_repvit_int8(batch=batch)
    else:
        raise SystemExit(f"unknown model {model!r}")
    rec = _Recorder()
    compile_graph(graph, batch=batch, schedule_fn=rec, conv_mode=conv_mode)
    return list(rec.problems.values())


def _precompile_one(args):
    problem, sched = args
    precompile(problem, sched)
    return 1


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--model", default="resnet18")
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--conv-mode", default="implicit")
    ap.add_argument("--budget", type=int, default=48)
    ap.add_argument("--precompile", action="store_true")
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--out", default=TUNED_PATH)
    ap.add_argument("--only", default="", help="substring filter on problem keys")
    args = ap.parse_args(argv)

    probs = [p for p in model_problems(args.model, args.batch, args.conv_mode)
             if args.only in problem_key(p)]
    print(f"{len(probs)} problems", flush=True)
    if args.precompile:
        work = [(p, s) for p in probs for s in problem_candidates(p, budget=args.budget)]
        t0 = time.time()
        with ProcessPoolExecutor(args.jobs) as pool:
            for i, _ in enumerate(pool.map(_precompile_one, work, chunksize=2), 1):
                if i % 25 == 0:
                    print(f"  compiled {i}/{len(work)} ({time.time() - t0:.0f} s)", flush=True)
        print(f"precompiled {len(work)} candidate modules in {time.time() - t0:.0f} s")
        return 0

    from mdlc_amd.codegen.hip.hiprtc_runtime import HipContext

    ctx = HipContext(0)
    cache = AutotuneCache(args.out)
    for p in probs:
        t0 = time.time()
        res = tune_problem(p, budget=args.budget, ctx=ctx)
        if p["kind"] == "qdw":
            d = default_qdw_schedule(p["M"]).key_full()
        else:
            d = (default_qschedule if is_int8(p) else default_schedule)(p["M"], p["N"], p["K"]).key_full()
        dflt = next((m for k, m in res.ranking if k == d), float("nan"))
        cache.put_key(res.key, res.best, res.best_metric, True)
        cache.save()
        flops = 2.0 * p["M"] * p["N"] * p["K"]
        print(f"{res.key:48s} best {res.best.key_full():40s} {res.best_metric * 1e3:9.1f} us "
              f"({flops / res.best_metric / 1e9:6.1f} TFLOP/s; default {dflt * 1e3:9.1f} us) "
              f"[{res.n_evaluated} cands, {len(res.rejected)} rejected, {time.time() - t0:.1f} s]",
              flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
