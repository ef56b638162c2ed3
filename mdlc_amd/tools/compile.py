"""CLI: compile a model for the MI355X backend and report what the compiler did.

    python -m mdlc_amd.tools.compile resnet18 --batch 32 --report
    python -m mdlc_amd.tools.compile mobilenetv2 --emit out.hip
    python -m mdlc_amd.tools.compile repvit_int8 --batch 32 --tune --cache my_schedules.json
    python -m mdlc_amd.tools.compile micro:784x128x1152 --run

The reference's CLI (mdlc/tools/compile.py:15-51) takes an ``.onnx`` path and
offers ``--report``, ``--emit FILE``, ``--tune`` and ``--no-verify``; the same
flags mean the same here. A model is an ``.onnx`` path (read by the
package's own protobuf reader) or the name of an IR-direct builder
(``resnet18``, ``mobilenetv2``, ``repvit_int8``, ``micro:MxNxK``). ``--emit`` writes the hipRTC translation
unit; ``--tune`` measures schedules on the device when one is visible (the
cost model ranks them otherwise) and saves the cache; ``--run`` executes one
forward on the device and prints its time.
"""

from __future__ import annotations

import argparse
import sys


def build_model(name: str, batch: int):
    """(graph, feeds) for a builtin model name."""
    if name.startswith("micro:"):
        from mdlc_amd.tools.micro_gemm import build_micro_gemm

        M, N, K = (int(v) for v in name.split(":", 1)[1].lower().split("x"))
        return build_micro_gemm(M, N, K)
    if name == "resnet18":
        from mdlc_amd.tools.build_resnet18 import build_resnet18 as build, make_input
    elif name == "mobilenetv2":
        from mdlc_amd.tools.build_mobilenetv2 import build_mobilenetv2 as build, make_input
    elif name == "repvit_int8":
        from mdlc_amd.tools.build_repvit_int8 import build_repvit_int8 as build, make_input
    else:
        raise SystemExit(f"unknown model {name!r}: use resnet18, mobilenetv2, repvit_int8, "
                         "micro:MxNxK or an .onnx path")
    return build(batch=batch), {"input": make_input(batch)}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="mdlc_amd: fused-group compiler for MI355X (gfx950)")
    ap.add_argument("model", help="resnet18 | mobilenetv2 | repvit_int8 | micro:MxNxK | path.onnx")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--report", action="store_true", help="print the full compile report")
    ap.add_argument("--emit", metavar="FILE", help="write the generated HIP source to FILE")
    ap.add_argument("--tune", action="store_true", help="autotune GEMM/conv schedules")
    ap.add_argument("--cache", default="", help="autotune JSON cache (default: the shipped "
                    "gfx950 schedules when not tuning, a new cache file when tuning)")
    ap.add_argument("--budget", type=int, default=24, help="candidates measured per problem")
    ap.add_argument("--conv-mode", default="implicit", choices=["implicit", "im2col"])
    ap.add_argument("--winograd", default="auto", choices=["auto", "always", "never"],
                    help="3x3 stride-1 convs as Winograd F(2x2, 3x3): where its grid fills half "
                         "the CUs (auto), always, or never (the implicit GEMM)")
    ap.add_argument("--no-fold", action="store_true",
                    help="keep the reference's fused groups (no residual / int8 epilogue folds)")
    ap.add_argument("--no-verify", action="store_true",
                    help="accepted for compatibility: structural verification always runs after "
                         "each pass; numerical verification needs the test oracle")
    ap.add_argument("--run", action="store_true", help="run one forward on the device and time it")
    ap.add_argument("--save-outputs", default="", metavar="NPZ",
                    help="with --run: write the graph outputs (and the feeds) to an .npz file")
    args = ap.parse_args(argv)

    from mdlc_amd.compiler import compile_graph, compile_onnx

    schedule_fn = None
    tuner = None
    if args.tune or args.cache:
        from mdlc_amd.autotuner.tuner import AutotuneCache, Tuner
        from mdlc_amd.codegen.hip.hiprtc_runtime import HipContext, hip_available

        ctx = HipContext(0) if (args.tune and hip_available()) else None
        path = args.cache or ("mdlc_amd_autotune.json" if args.tune else "")
        tuner = Tuner(AutotuneCache(path), ctx=ctx, budget=args.budget, tune_misses=args.tune)
        schedule_fn = tuner

    kw = dict(batch=args.batch, schedule_fn=schedule_fn, conv_mode=args.conv_mode,
              winograd={"auto": "auto", "always": True, "never": False}[args.winograd])
    if args.no_fold:
        kw.update(fuse_residual=False, fuse_int8_epilogues=False)
    if args.model.endswith(".onnx"):
        from mdlc_amd.frontend import OnnxDecodeError

        try:
            compiled = compile_onnx(args.model, **kw)
        except (NotImplementedError, OnnxDecodeError, OSError) as exc:
            print(f"error: {exc}", file=sys.stderr)
            return 2
        feeds = compiled.feeds
    else:
        graph, feeds = build_model(args.model, args.batch)
        compiled = compile_graph(graph, feeds=feeds, **kw)

    if args.report or not (args.emit or args.run):
        print(compiled.report())

    if tuner is not None and args.tune:
        tuner.cache.save()
        how = "measured on the device" if tuner.ctx is not None else "ranked by the cost model"
        print(f"\nautotune cache: {len(tuner.cache.entries)} problems ({how}) -> {tuner.cache.path}")

    if args.emit:
        with open(args.emit, "w") as f:
            f.write(compiled.module.sources())
        print(f"\nwrote generated HIP ({len(compiled.module.kernels)} kernels, "
              f"{len(compiled.module.plan)} launches) to {args.emit}")

    if args.run:
        from mdlc_amd.codegen.hip.hip_executor import HipExecutor

        ex = HipExecutor(compiled.module)
        try:
            res = ex.run(feeds, timing=True)
        finally:
            ex.close()
        shapes = ", ".join(f"{k}{tuple(v.shape)}" for k, v in res["outputs"].items())
        print(f"\nran on the device: {res['ms']:.3f} ms ({shapes})")
        if args.save_outputs:
            import numpy as np

            np.savez(args.save_outputs, **{f"out:{k}": v for k, v in res["outputs"].items()},
                     **{f"in:{k}": np.asarray(v) for k, v in feeds.items()})
            print(f"wrote outputs and feeds to {args.save_outputs}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
