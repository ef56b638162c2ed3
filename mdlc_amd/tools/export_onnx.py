"""CLI: write a builtin model as an ONNX file.

    python -m mdlc_amd.tools.export_onnx resnet18 --batch 1 --out resnet18.onnx

The reference's exporters (mdlc/tools/build_resnet18.py:14-38,
build_mobilenetv2.py:14-47) write torchvision models with random weights to
``.onnx`` for the compiler and the benchmark. Here the same networks come
from the IR-direct builders (random weights in the benchmark
distributions), serialized by ``mdlc_amd.frontend.onnx_export``; the file
compiles with ``python -m mdlc_amd.tools.compile model.onnx``.
"""

from __future__ import annotations

import argparse


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="write a builtin model as an ONNX file")
    ap.add_argument("model", help="resnet18 | mobilenetv2 | micro:MxNxK")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--out", default="", help="output path (default: <model>.onnx)")
    args = ap.parse_args(argv)

    from mdlc_amd.frontend.onnx_export import export_onnx
    from mdlc_amd.tools.compile import build_model

    if args.model == "repvit_int8":
        raise SystemExit("repvit_int8 uses this backend's quantized operators (QConv, QLut, ...), "
                         "which are not ONNX operators")
    graph, _ = build_model(args.model, args.batch)
    path = args.out or args.model.replace(":", "_") + ".onnx"
    data = export_onnx(graph, path)
    print(f"wrote {path} ({len(data)} bytes, {len(graph.nodes)} nodes)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
