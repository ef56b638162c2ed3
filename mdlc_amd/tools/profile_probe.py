"""A plain device copy of known size, for calibrating hardware byte counters.

    python -m mdlc_amd.tools.profile_probe --mib 256 [--iters 5]

Runs the backend's ``copy_bytes`` kernel (the same one reshaping views
lower to) over a ``--mib`` MiB buffer ``--iters`` times. Under
``rocprofv3 --pmc FETCH_SIZE`` (or ``WRITE_SIZE``) each dispatch should read
(write) exactly that many bytes; the ratio of the counter to the true size is
the scale factor applied to the counters of the kernels being measured.
"""

from __future__ import annotations

import argparse

import numpy as np


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=256)
    ap.add_argument("--iters", type=int, default=5)
    args = ap.parse_args(argv)

    from mdlc_amd.codegen.hip.hip_executor import HipExecutor
    from mdlc_amd.compiler import compile_graph
    from mdlc_amd.tools.graph_builder import GraphBuilder

    n = args.mib * 1024 * 1024 // 4
    b = GraphBuilder("copy_probe")
    b.input("x", (n,))
    b.node("Identity", ["x"], "y")
    b.output("y")
    feeds = {"x": np.arange(n, dtype=np.float32)}
    c = compile_graph(b.graph(), feeds=feeds)
    ex = HipExecutor(c.module)
    try:
        ex._upload_feeds(feeds)
        ex.plan.run(args.iters)
        ex.ctx.synchronize()
        ok = bool(np.array_equal(ex.read("y"), feeds["x"]))
        ms = ex.plan.time_ms(0, args.iters)
    finally:
        ex.close()
    kib = n * 4 / 1024
    print(f"copy_probe: {kib:.0f} KiB read + {kib:.0f} KiB written per dispatch, "
          f"{ms * 1e3:.1f} us, {2 * n * 4 / ms / 1e6:.0f} GB/s, exact={ok}")
    return 0 if ok else 1


if __name__ == "__main__":
    raise SystemExit(main())
