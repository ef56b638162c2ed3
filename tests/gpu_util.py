"""Helpers shared by the GPU parity tests: compile a graph for the device,
run it, and compare against the oracle."""

from __future__ import annotations

import numpy as np

from mdlc_amd.compiler import compile_graph
from mdlc_amd.codegen.hip.hip_executor import HipExecutor
from mdlc_amd.testing import DEVICE_TENSOR, compare_arrays, tolerance_ratio
from oracle.reference import run_reference


def device_run(graph, feeds, *, schedule_fn=None, conv_mode="implicit", ctx=None, all_tensors=False,
               **compile_kw):
    """Compile ``graph`` (fused by the default pipeline) and run it on the
    device. Returns (compiled, device values, oracle values)."""
    c = compile_graph(graph, feeds=feeds, schedule_fn=schedule_fn, conv_mode=conv_mode, **compile_kw)
    ex = HipExecutor(c.module, ctx)
    try:
        got = ex.run_all(feeds) if all_tensors else ex.run(feeds)["outputs"]
    finally:
        ex.close()
    want = run_reference(c.graph, feeds, return_all=all_tensors)
    return c, got, want


def assert_close(name, got, want, tol=DEVICE_TENSOR, vacuous_ok=False):
    if np.issubdtype(np.asarray(want).dtype, np.integer):
        assert np.array_equal(got, want), f"{name}: integer mismatch " \
            f"({int(np.sum(np.asarray(got) != np.asarray(want)))} elements differ)"
        return
    r = compare_arrays(name, got, want, rtol=tol.rtol, atol=tol.atol)
    if not r.ok and vacuous_ok and "VACUOUS" in r.detail:
        return
    assert r.ok, f"{r} ratio={tolerance_ratio(got, want, rtol=tol.rtol, atol=tol.atol):.3f}"
