"""Vendor-library yardsticks on the same device: what PyTorch-ROCm reaches
with MIOpen (conv) and hipBLASLt (GEMM) on the workloads this backend is
measured on.

    python -m mdlc_amd.tools.vendor_baseline            # all three
    python -m mdlc_amd.tools.vendor_baseline --only resnet18

These numbers put the generated kernels' throughput in context; they are not
part of the compiled path and nothing in the backend calls PyTorch's
convolution or matmul. ResNet-18 is built in ``torch.nn`` with BatchNorm
already folded into the conv bias (the same arithmetic the fused groups do),
fp32 with TF32-style reduced precision disabled, NCHW and channels-last, eager
and replayed from a captured graph. The GEMMs are ``torch.mm`` in fp32 and
``torch._int_mm`` (int8 x int8 -> int32).
"""

from __future__ import annotations

import argparse
import json
import time


def _time(fn, iters: int, warmup: int) -> float:
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / iters


def resnet18(batch: int, iters: int):
    import torch
    from torch import nn

    class Block(nn.Module):
        def __init__(self, cin, cout, stride):
            super().__init__()
            self.c1 = nn.Conv2d(cin, cout, 3, stride, 1)
            self.c2 = nn.Conv2d(cout, cout, 3, 1, 1)
            self.proj = nn.Conv2d(cin, cout, 1, stride, 0) if (stride != 1 or cin != cout) else None

        def forward(self, x):
            y = torch.relu(self.c1(x))
            y = self.c2(y)
            return torch.relu(y + (self.proj(x) if self.proj is not None else x))

    layers = [nn.Conv2d(3, 64, 7, 2, 3), nn.ReLU(), nn.MaxPool2d(3, 2, 1)]
    cin = 64
    for cout, stride in ((64, 1), (128, 2), (256, 2), (512, 2)):
        layers += [Block(cin, cout, stride), Block(cout, cout, 1)]
        cin = cout
    layers += [nn.AdaptiveAvgPool2d(1), nn.Flatten(), nn.Linear(512, 1000)]
    out = {}
    for fmt in ("nchw", "channels_last"):
        mf = torch.channels_last if fmt == "channels_last" else torch.contiguous_format
        model = nn.Sequential(*layers).cuda().eval().to(memory_format=mf)
        x = torch.randn(batch, 3, 224, 224, device="cuda").to(memory_format=mf)
        with torch.no_grad():
            eager = _time(lambda: model(x), iters, 5)
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for _ in range(3):
                    model(x)
            torch.cuda.current_stream().wait_stream(s)
            with torch.cuda.graph(g):
                model(x)
            graph = _time(g.replay, iters, 5)
        out[fmt] = {"eager_img_s": batch / eager, "graph_img_s": batch / graph,
                    "graph_ms": graph * 1e3}
    return out


def gemms(iters: int):
    import torch

    out = {}
    for n in (4096, 8192):
        a = torch.randn(n, n, device="cuda")
        b = torch.randn(n, n, device="cuda")
        t = _time(lambda: torch.mm(a, b), iters, 3)
        out[f"fp32_{n}"] = {"tflops": 2 * n ** 3 / t / 1e12, "ms": t * 1e3}
        ai = torch.randint(-127, 128, (n, n), device="cuda", dtype=torch.int8)
        bi = torch.randint(-127, 128, (n, n), device="cuda", dtype=torch.int8)
        t = _time(lambda: torch._int_mm(ai, bi), iters, 3)
        out[f"int8_{n}"] = {"tops": 2 * n ** 3 / t / 1e12, "ms": t * 1e3}
        del a, b, ai, bi
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--only", choices=["resnet18", "gemm"], default=None)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--iters", type=int, default=30)
    args = ap.parse_args(argv)

    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    res = {"device": torch.cuda.get_device_name(0), "torch": torch.__version__}
    if args.only in (None, "resnet18"):
        res[f"resnet18_b{args.batch}"] = resnet18(args.batch, args.iters)
        print(json.dumps(res), flush=True)
    if args.only in (None, "gemm"):
        res["gemm"] = gemms(args.iters)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
