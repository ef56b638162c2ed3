"""The allocation-free plan runner (mdlc_plan_run_static): the same plan run
on the library's static per-GPU scratch instead of a workspace in the
executor's arena gives bit-identical results, on two calls in a row (the
second on a smaller problem), and plans whose workspace does not fit are
refused on the host before anything is launched."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from mdlc_amd.codegen.hip import hiprtc_runtime as R
from mdlc_amd.codegen.hip.hip_executor import HipExecutor
from mdlc_amd.codegen.schedule import MfmaSchedule
from mdlc_amd.compiler import compile_graph
from mdlc_amd.tools.build_resnet18 import build_resnet18, make_input
from mdlc_amd.tools.micro_gemm import build_micro_gemm

pytestmark = pytest.mark.gpu


def _both(c, feeds, ctx):
    """Every tensor the plan writes, from the arena-workspace run and from
    the static-scratch run."""
    out = []
    for static in (False, True):
        ex = HipExecutor(c.module, ctx, static_scratch=static)
        try:
            assert (ex.ws_bytes > 0) == static
            chained = ex.run(feeds)["outputs"]
            every = ex.run_all(feeds)
        finally:
            ex.close()
        out.append((chained, every))
    return out


def test_static_scratch_matches_the_arena_workspace(hip_ctx):
    # first call: ResNet-18 at batch 32 on the implicit GEMM (split-K and
    # stream-K workspaces, 32 MB)
    x = make_input(32)
    c = compile_graph(build_resnet18(batch=32), feeds={"input": x}, winograd=False)
    kinds = {l.kind for l in c.module.plan}
    assert {"splitk_reduce", "streamk_fixup"} <= kinds
    (ca, ea), (cs, es) = _both(c, {"input": x}, hip_ctx)
    np.testing.assert_array_equal(cs["logits"], ca["logits"])
    assert ea.keys() == es.keys() and "logits" in ea
    for t in ea:
        np.testing.assert_array_equal(es[t], ea[t], err_msg=t)

    # second call, smaller: one micro GEMM with a split-K workspace
    g, feeds = build_micro_gemm(784, 128, 1152)
    c2 = compile_graph(g, feeds=feeds, schedule_fn=lambda n, mnk: MfmaSchedule(64, 64, 16, 2, 2, 32, True, 4))
    assert "splitk_reduce" in {l.kind for l in c2.module.plan}
    (ca, ea), (cs, es) = _both(c2, feeds, hip_ctx)
    np.testing.assert_array_equal(cs["C"], ca["C"])
    for t in ea:
        np.testing.assert_array_equal(es[t], ea[t], err_msg=t)


def test_static_scratch_limits_are_host_errors(hip_ctx):
    # a workspace above the static scratch is refused by the executor ...
    c = compile_graph(build_resnet18(batch=32), feeds={"input": make_input(32)}, conv_mode="im2col")
    with pytest.raises(R.HipError, match="exceeds the static scratch"):
        HipExecutor(c.module, hip_ctx, static_scratch=True)
    # ... and by the entry point itself, before any launch; a plan without a
    # workspace of its own is refused by the arena runner
    g, feeds = build_micro_gemm(784, 128, 1152)
    c2 = compile_graph(g, feeds=feeds, schedule_fn=lambda n, mnk: MfmaSchedule(64, 64, 16, 2, 2, 32, True, 4))
    ex = HipExecutor(c2.module, hip_ctx, static_scratch=True)
    assert ex.ws_bytes > 0
    try:
        recs = ex.launch_records
        big = R.Plan(recs, (0, R.STATIC_SCRATCH_BYTES + 256))
        with pytest.raises(R.HipError, match="exceeds the static scratch"):
            big.run_static(1)
        with pytest.raises(R.HipError, match="no workspace bound"):
            big.run(1)
        big.close()
    finally:
        ex.close()
    assert R.lib().mdlc_sync() == 0
