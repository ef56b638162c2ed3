"""Device parity of each gfx950 kernel template against the NumPy oracle.

Mirrors the reference's kernel tests (tests/test_codegen_kernels.py:18-120:
GEMM at 65x48x33 over several schedules and epilogues, seed 0; im2col at
3x9x9 k3 s1 p1, seed 1; conv via im2col + GEMM, seed 2; relu(a+b)*c over 256
elements, seed 3) but runs the kernels on the MI355X, adds batch N in
{1, 2, 8} for every conv (the reference's batch>1 gap), and holds every
float32 tensor to rtol 1e-4 / atol 1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest

from gpu_util import assert_close, device_run
from mdlc_amd.codegen.schedule import MfmaSchedule, smallc_tile
from mdlc_amd.ir import Node
from mdlc_amd.testing import BITWISE, DEVICE_TENSOR
from mdlc_amd.tools.graph_builder import GraphBuilder
from mdlc_amd.tools.micro_gemm import SHAPES, build_micro_gemm

pytestmark = pytest.mark.gpu

SCHEDULES = [
    MfmaSchedule(),                                   # 128x128x16, 2x2 waves, 32x32x2
    MfmaSchedule(64, 64, 16, 2, 2, 32, True),
    MfmaSchedule(32, 32, 8, 1, 1, 32, True),
    MfmaSchedule(64, 64, 16, 2, 2, 16, True),         # 16x16x4 MFMA
    MfmaSchedule(128, 64, 32, 2, 2, 16, False),       # single buffered
    MfmaSchedule(256, 128, 16, 4, 2, 32, True),
    MfmaSchedule(64, 64, 16, 2, 2, 32, True, 3),       # split-K, ragged last slice
    MfmaSchedule(32, 32, 16, 1, 1, 16, True, 2),       # split-K with 16x16x4
    MfmaSchedule(32, 32, 16, 1, 1, 16, True, 1, True),  # stream-K: every tile in pieces
    MfmaSchedule(64, 64, 16, 2, 2, 32, False, 1, True),
    MfmaSchedule(64, 64, 16, 2, 2, 32, True, 1, False, 2),      # K loop unrolled by two
    MfmaSchedule(64, 64, 16, 2, 2, 32, True, 3, False, 2),      # ... with split-K slices
    MfmaSchedule(32, 32, 16, 1, 1, 16, True, 1, True, 2),       # ... with stream-K pieces
    MfmaSchedule.wsplit(16, 16, 4),                            # K over the waves of a workgroup
    MfmaSchedule.wsplit(32, 32, 16, 2),
    MfmaSchedule.wsplit(16, 32, 8, 2),
    MfmaSchedule.wsplit(16, 16, 8, 8),
    MfmaSchedule.wsplit(32, 16, 4, 1, True),                   # weights K-contiguous per column
    MfmaSchedule.wsplit(64, 16, 4, 2),                         # 64-row tile
    MfmaSchedule.wsplit(16, 64, 8, 4, True),                   # 64-column tile, deep stages
    MfmaSchedule.wsplit(16, 16, 4, 2, True, 3),                # ... and K over 3 workgroups
    MfmaSchedule.wsplit(32, 32, 8, 1, False, 2),
]


def _gemm_graph(M, N, K, act, bias, seed=0, trans_b=False):
    rng = np.random.default_rng(seed)
    b = GraphBuilder("g")
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    b.input("A", (M, K))
    b.const("B", B.T.copy() if trans_b else B)
    ins = ["A", "B"]
    if bias:
        b.const("bias", rng.standard_normal(N).astype(np.float32))
        ins.append("bias")
    out = "C" if act is None else "pre"
    b.node("Gemm", ins, out, transB=1 if trans_b else 0)
    if act is not None:
        b.node(act, [out], "C")
    b.output("C")
    return b.graph(), {"A": A}


@pytest.mark.parametrize("sched", SCHEDULES, ids=lambda s: s.key_full())
@pytest.mark.parametrize("act,bias", [("Relu", True), (None, False), ("Sigmoid", True)])
def test_gemm_kernel_matches_oracle(sched, act, bias, hip_ctx):
    assert sched.is_valid()
    g, feeds = _gemm_graph(65, 48, 33, act, bias)          # non-tile multiples
    c, got, want = device_run(g, feeds, schedule_fn=lambda n, mnk: sched, ctx=hip_ctx)
    assert c.module.fallbacks() == []
    assert_close("C", got["C"], want["C"])


@pytest.mark.parametrize("M,N,K", [(1, 1000, 512), (7, 13, 5), (130, 260, 64), (33, 1001, 77)])
def test_gemm_transb_and_ragged_shapes(M, N, K, hip_ctx):
    g, feeds = _gemm_graph(M, N, K, "Relu", True, seed=5, trans_b=True)
    _, got, want = device_run(g, feeds, ctx=hip_ctx)
    assert_close("C", got["C"], want["C"])


@pytest.mark.parametrize("sched", [MfmaSchedule.wsplit(16, 16, 4, 2), MfmaSchedule.wsplit(32, 16, 8, 1, True),
                                   MfmaSchedule.wsplit(16, 64, 4, 4, True),
                                   MfmaSchedule.wsplit(16, 32, 4, 1, True, 4)], ids=lambda s: s.key_full())
@pytest.mark.parametrize("M,N,K", [(1, 1000, 512), (7, 13, 5), (33, 1001, 77), (5, 70, 300)])
@pytest.mark.parametrize("trans_b", [False, True])
def test_wave_split_ragged_shapes(M, N, K, trans_b, sched, hip_ctx):
    """The wave-split kernel's out-of-range reads (rows past M, columns past
    N, k past K inside a row, steps past a wave's share) all read zero."""
    g, feeds = _gemm_graph(M, N, K, "Relu", True, seed=6, trans_b=trans_b)
    c, got, want = device_run(g, feeds, ctx=hip_ctx, schedule_fn=lambda n, mnk: sched)
    assert [l.kind for l in c.module.plan][0] == "gemm_ws"
    assert_close("C", got["C"], want["C"])


@pytest.mark.parametrize("M,N,K", SHAPES, ids=lambda v: str(v))
def test_micro_gemm_shapes(M, N, K, hip_ctx):
    """The fused GEMM+bias+ReLU micro workload at ResNet-18's batch-1 shapes."""
    g, feeds = build_micro_gemm(M, N, K)
    c, got, want = device_run(g, feeds, ctx=hip_ctx)
    assert [n.op_type for n in c.graph.nodes] == ["FusedGemmAct"]
    assert_close("C", got["C"], want["C"])


@pytest.mark.parametrize("sched", [MfmaSchedule.wsplit(16, 16, 8), MfmaSchedule.wsplit(32, 16, 16, 2),
                                   MfmaSchedule.wsplit(16, 32, 4, 2), MfmaSchedule.wsplit(16, 16, 16, 8),
                                   MfmaSchedule.wsplit(32, 16, 4, 4), MfmaSchedule.wsplit(16, 16, 8, 2, True),
                                   MfmaSchedule.wsplit(32, 32, 4, 1, True), MfmaSchedule.wsplit(16, 64, 8),
                                   MfmaSchedule.wsplit(64, 32, 4, 2), MfmaSchedule.wsplit(16, 16, 8, 2, True, 8),
                                   MfmaSchedule.wsplit(64, 16, 4, 4, True, 12)], ids=lambda s: s.key_full())
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_micro_gemm_wave_split(M, N, K, sched, hip_ctx):
    """The wave-split kernel on the micro shapes (16-byte A loads, K % 16 ==
    0) against the oracle: one launch, or with K also split over workgroups
    the partial launch and the ordered reduce."""
    g, feeds = build_micro_gemm(M, N, K)
    c, got, want = device_run(g, feeds, ctx=hip_ctx, schedule_fn=lambda n, mnk: sched)
    kinds = [l.kind for l in c.module.plan]
    assert kinds == (["gemm_ws", "splitk_reduce"] if sched.SK > 1 else ["gemm_ws"])
    assert_close("C", got["C"], want["C"])


def _conv_graph(n, c, h, w, oc, k, s, p, act="Relu", bias=True, seed=2, group=1):
    rng = np.random.default_rng(seed)
    b = GraphBuilder("conv")
    b.input("x", (n, c, h, w))
    b.const("w", (rng.standard_normal((oc, c // group, k, k)) * np.sqrt(2.0 / (c // group * k * k)))
            .astype(np.float32))
    ins = ["x", "w"]
    if bias:
        b.const("b", rng.standard_normal(oc).astype(np.float32) * 0.1)
        ins.append("b")
    out = "y" if act is None else "pre"
    b.node("Conv", ins, out, kernel_shape=[k, k], strides=[s, s], pads=[p] * 4, group=group)
    if act == "Clip":
        b.const("lo", np.float32(0.0))
        b.const("hi", np.float32(6.0))
        b.node("Clip", [out, "lo", "hi"], "y")
    elif act is not None:
        b.node(act, [out], "y")
    b.output("y")
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    return b.graph(), {"x": x}


CONV_CASES = [
    # n, c, h, w, oc, k, s, p
    (1, 3, 9, 9, 8, 3, 1, 1),
    (2, 3, 9, 9, 8, 3, 1, 1),
    (8, 3, 9, 9, 8, 3, 1, 1),
    (2, 3, 23, 23, 64, 7, 2, 3),
    (2, 16, 14, 14, 32, 3, 2, 1),
    (2, 16, 14, 14, 32, 1, 2, 0),
    (1, 64, 7, 7, 128, 3, 1, 1),
]


@pytest.mark.parametrize("mode", ["implicit", "im2col", "implicit-gemm", "winograd"])
@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: "x".join(map(str, c)))
def test_conv_matches_oracle(case, mode, hip_ctx):
    """Implicit mode takes the direct small-channel kernel for C <= 4;
    "implicit-gemm" keeps those convs on the implicit-GEMM gather; "winograd"
    (the default) runs 3x3 stride-1 convs of more channels as Winograd."""
    g, feeds = _conv_graph(*case)
    c, got, want = device_run(g, feeds, conv_mode="im2col" if mode == "im2col" else "implicit",
                              ctx=hip_ctx, small_conv=mode != "implicit-gemm",
                              winograd=mode == "winograd")
    assert [n.op_type for n in c.graph.nodes] == ["FusedConvAct"]
    kinds = [l.kind for l in c.module.plan]
    assert ("conv_smallc" in kinds) == (mode in ("implicit", "winograd") and case[1] <= 4)
    assert ("wino" in kinds) == (mode == "winograd" and case[1] > 4 and case[5] == 3 and case[6] == 1)
    assert_close("y", got["y"], want["y"])


WS_CONV_CASES = [
    # n, c, h, w, oc, k, s, p: Cin % 16 == 0 (taps whole per 16-deep K step)
    (1, 16, 9, 9, 24, 3, 1, 1),
    (2, 32, 7, 7, 48, 3, 1, 1),          # tiles cross images (49 pixels an image)
    (3, 16, 14, 14, 40, 3, 2, 1),
    (2, 64, 14, 14, 72, 1, 2, 0),
    (1, 128, 5, 5, 96, 3, 1, 1),
]


@pytest.mark.parametrize("sched", [MfmaSchedule.wsplit(16, 16, 4, 1), MfmaSchedule.wsplit(32, 16, 8, 2),
                                   MfmaSchedule.wsplit(16, 64, 4, 2, False, 3),
                                   MfmaSchedule.wsplit(64, 32, 8, 1, False, 2)],
                         ids=lambda s: s.key_full())
@pytest.mark.parametrize("case", WS_CONV_CASES, ids=lambda c: "x".join(map(str, c)))
def test_conv_wave_split(case, sched, hip_ctx):
    """The wave-split kernel on tap-major implicit-GEMM convolutions (padding
    taps, stride 2, 1x1, columns of one tile in several images), with the
    bias/ReLU epilogue, or K also split over workgroups and the reduce."""
    g, feeds = _conv_graph(*case)
    c, got, want = device_run(g, feeds, ctx=hip_ctx, winograd=False, small_conv=False,
                              schedule_fn=lambda n, mnk: sched)
    kinds = [l.kind for l in c.module.plan]
    assert kinds == (["conv_ws", "splitk_reduce"] if sched.SK > 1 else ["conv_ws"])
    assert_close("y", got["y"], want["y"])


def test_resnet18_b1_wave_split_convs(hip_ctx):
    """ResNet-18 batch 1 with every conv of 16 or more input channels on the
    wave-split kernel (residual adds folded into its epilogue or the split-K
    reduce), each fused group in isolation on the oracle's inputs."""
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor
    from mdlc_amd.compiler import compile_graph
    from mdlc_amd.tools.build_resnet18 import build_resnet18, make_input
    from oracle.reference import run_reference

    def fn(node, mnk):
        M, N, K = mnk
        return MfmaSchedule.wsplit(16, 32, 8, 1, False, 4 if K >= 2304 else 1)

    x = make_input(1)
    c = compile_graph(build_resnet18(batch=1, calibrate=True), feeds={"input": x}, schedule_fn=fn,
                      winograd=False)
    assert sum(l.kind == "conv_ws" for l in c.module.plan) == 19
    want = run_reference(c.graph, {"input": x}, return_all=True)
    ex = HipExecutor(c.module, hip_ctx)
    try:
        ex._upload_feeds({"input": x})
        got = ex.run_isolated(want)
    finally:
        ex.close()
    for t, v in got.items():
        assert_close(t, v, want[t])


SMALLC_CASES = [
    # n, c, h, w, oc, k, s, p, act, bias: every tile rule, ragged edges, OC not a multiple of 32
    (2, 3, 30, 30, 64, 7, 2, 3, "Relu", True),
    (1, 3, 17, 19, 32, 3, 2, 1, "Clip", True),
    (2, 1, 9, 9, 40, 3, 1, 1, None, False),
    (1, 4, 12, 20, 96, 5, 1, 2, "Relu", True),
    (2, 2, 15, 15, 24, 4, 2, 1, "Sigmoid", True),
    (3, 3, 40, 36, 70, 7, 2, 3, "Relu", False),
    (64, 3, 16, 16, 256, 3, 1, 1, "Relu", True),       # 8x16 blocks (>= 512 workgroups)
]


@pytest.mark.parametrize("case", SMALLC_CASES, ids=lambda c: "x".join(map(str, c[:8])))
def test_conv_small_channels_direct(case, hip_ctx):
    """The direct small-channel kernel (input patch in LDS, weights in
    registers, 32x32x2 MFMAs) against the oracle, and equal to a repeat run."""
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor
    from mdlc_amd.compiler import compile_graph
    from oracle.reference import run_reference

    *geo, act, bias = case
    g, feeds = _conv_graph(*geo, act=act, bias=bias)
    c = compile_graph(g, feeds=feeds)
    (launch,) = [l for l in c.module.plan if l.kind == "conv_smallc"]
    m = launch.meta
    assert m["tile"] == smallc_tile(geo[0], m["OC"], m["OH"], m["OW"])
    ex = HipExecutor(c.module, hip_ctx)
    try:
        y1 = ex.run(feeds)["outputs"]["y"]
        y2 = ex.run(feeds)["outputs"]["y"]
    finally:
        ex.close()
    assert_close("y", y1, run_reference(c.graph, feeds)["y"])
    np.testing.assert_array_equal(y1, y2)


@pytest.mark.parametrize("wgs", [1, 7])
def test_conv_small_channels_blocks_per_workgroup(wgs, hip_ctx, monkeypatch):
    """Fewer workgroups than output blocks: each steps through several blocks,
    prefetching the next patch while it computes (1 workgroup: every block in
    turn; 7: an uneven share, the last block partial)."""
    from mdlc_amd.codegen.hip import emit as E

    monkeypatch.setattr(E, "SMALLC_WGS", wgs)
    g, feeds = _conv_graph(3, 3, 37, 45, 64, 7, 2, 3)
    c, got, want = device_run(g, feeds, ctx=hip_ctx)
    (launch,) = [l for l in c.module.plan if l.kind == "conv_smallc"]
    assert launch.grid[0] == wgs
    assert_close("y", got["y"], want["y"])


def test_conv_small_channels_residual(hip_ctx):
    """A residual add folded into the direct small-channel conv's epilogue."""
    rng = np.random.default_rng(11)
    b = GraphBuilder("smallres")
    b.input("x", (2, 3, 20, 20))
    b.input("r", (2, 48, 10, 10))
    b.const("w", (rng.standard_normal((48, 3, 7, 7)) * 0.1).astype(np.float32))
    b.const("b", (rng.standard_normal(48) * 0.1).astype(np.float32))
    b.node("Conv", ["x", "w", "b"], "c", kernel_shape=[7, 7], strides=[2, 2], pads=[3, 3, 3, 3])
    b.node("Relu", ["c"], "y")
    b.node("Add", ["y", "r"], "s")
    b.node("Relu", ["s"], "z")
    b.output("z")
    feeds = {"x": rng.standard_normal((2, 3, 20, 20)).astype(np.float32),
             "r": rng.standard_normal((2, 48, 10, 10)).astype(np.float32)}
    c, got, want = device_run(b.graph(), feeds, ctx=hip_ctx)
    assert [l.kind for l in c.module.plan] == ["conv_smallc"]
    assert_close("z", got["z"], want["z"])


CONV_POOL_CASES = [   # (N, C, H, W, OC, K, S, P, activation, bias)
    (2, 3, 32, 32, 20, 7, 2, 3, "Relu", True),      # OC not a multiple of 16: masked channels
    (1, 3, 64, 64, 64, 7, 2, 3, "Relu", True),      # two column blocks: the carried column
    (1, 2, 32, 32, 16, 3, 1, 1, "Clip", False),
    (1, 1, 64, 32, 40, 5, 2, 2, None, True),
    (3, 3, 224, 224, 64, 7, 2, 3, "Relu", True),    # the ResNet stem's width, bands of 7 rows
]


@pytest.mark.parametrize("case", CONV_POOL_CASES, ids=lambda c: "x".join(map(str, c[:8])))
def test_conv_pool_fused(case, hip_ctx, monkeypatch):
    """The small-channel conv with the 3x3 stride-2 max pool after it in one
    launch, against the oracle's conv -> activation -> pool on the unfolded
    graph (rtol 1e-4 / atol 1e-5), and equal to a repeat run. The CU count is
    lowered so that small shapes take the fused kernel (the fold wants a band
    of pooled rows per CU)."""
    import mdlc_amd.codegen.schedule as S
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor
    from mdlc_amd.compiler import compile_graph
    from oracle.reference import run_reference
    from test_conv_pool import _graph as conv_pool_graph

    monkeypatch.setattr(S, "CUS", 2)
    n, c_in, h, w, oc, k, s, p, act, bias = case
    g, feeds = conv_pool_graph(n, c_in, h, w, oc, k, s, p, act=act, bias=bias)
    c = compile_graph(g.clone(), feeds=feeds)
    assert [l.kind for l in c.module.plan] == ["conv_pool"]
    ex = HipExecutor(c.module, hip_ctx)
    try:
        z1 = ex.run(feeds)["outputs"]["z"]
        z2 = ex.run(feeds)["outputs"]["z"]
    finally:
        ex.close()
    assert_close("z", z1, run_reference(g, feeds)["z"])
    np.testing.assert_array_equal(z1, z2)


@pytest.mark.parametrize("mode", ["implicit", "im2col"])
@pytest.mark.parametrize("sk", [2, 4, 5])
@pytest.mark.parametrize("case", [CONV_CASES[2], CONV_CASES[4], CONV_CASES[6]],
                         ids=lambda c: "x".join(map(str, c)))
def test_conv_split_k(case, sk, mode, hip_ctx):
    """Split-K (partial slices + ordered reduce launch): correct on the first
    run and on repeated runs of one executor, with a different input in
    between (the workspace is fully rewritten every run)."""
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor
    from mdlc_amd.compiler import compile_graph
    from oracle.reference import run_reference

    sched = MfmaSchedule(64, 64, 16, 2, 2, 32, True, sk)
    g, feeds = _conv_graph(*case)
    c = compile_graph(g, feeds=feeds, conv_mode=mode, schedule_fn=lambda n, mnk: sched,
                      small_conv=False, winograd=False)
    (launch,) = [l for l in c.module.plan if l.kind in ("conv", "gemm")]
    assert launch.meta["ksplit"] > 1 and launch.grid[0] % launch.meta["ksplit"] == 0
    assert [l.kind for l in c.module.plan][-1] == "splitk_reduce"
    feeds2 = {"x": (feeds["x"][::-1] * 0.5).copy()}
    ex = HipExecutor(c.module, hip_ctx)
    try:
        for f in (feeds, feeds2, feeds):
            got = ex.run(f)["outputs"]
            assert_close("y", got["y"], run_reference(c.graph, f)["y"])
    finally:
        ex.close()


# Implicit-GEMM schedules covering every gather/staging shape: threads per
# column 1..16, k rows per thread 1..32 (scalar, pair and quad LDS stores),
# both MFMA shapes, single and double buffering.
CONV_SCHEDULES = [
    MfmaSchedule(64, 64, 16, 2, 2, 32, True),       # 4 threads/column, 4 rows each
    MfmaSchedule(128, 32, 16, 4, 2, 16, True),      # 16 threads/column, 1 row each
    MfmaSchedule(128, 64, 16, 4, 2, 16, True),      # 8 threads/column, 2 rows each
    MfmaSchedule(64, 64, 32, 4, 2, 16, True),       # 8 threads/column, 4 rows each
    MfmaSchedule(32, 128, 32, 1, 2, 32, False),     # 1 thread/column, 32 rows, single buffered
    MfmaSchedule(64, 64, 32, 4, 2, 16, True, 1, False, 2),   # K loop unrolled by two
]


@pytest.mark.parametrize("sched", CONV_SCHEDULES, ids=lambda s: s.key())
@pytest.mark.parametrize("case", [CONV_CASES[3], CONV_CASES[4], CONV_CASES[6]],
                         ids=lambda c: "x".join(map(str, c)))
def test_conv_gather_schedules(case, sched, hip_ctx):
    """Channel-major (C % BK != 0) and tap-major (C % BK == 0) gathers."""
    assert sched.conv_valid()
    g, feeds = _conv_graph(*case)
    c, got, want = device_run(g, feeds, conv_mode="implicit", ctx=hip_ctx,
                              schedule_fn=lambda n, mnk: sched, small_conv=False, winograd=False)
    (launch,) = [l for l in c.module.plan if l.kind == "conv"]
    assert launch.meta["k_order"] == ("tap" if case[1] % sched.BK == 0 else "channel")
    assert_close("y", got["y"], want["y"])


def _conv_residual_graph(post, res_first, seed=9):
    rng = np.random.default_rng(seed)
    b = GraphBuilder("cres")
    b.input("x", (2, 32, 10, 10))
    b.input("r", (2, 48, 10, 10))
    b.const("w", (rng.standard_normal((48, 32, 3, 3)) * 0.08).astype(np.float32))
    b.const("b", (rng.standard_normal(48) * 0.1).astype(np.float32))
    b.node("Conv", ["x", "w", "b"], "c", kernel_shape=[3, 3], pads=[1, 1, 1, 1])
    b.node("Relu", ["c"], "y")
    b.node("Add", ["r", "y"] if res_first else ["y", "r"], "s")
    if post == "relu":
        b.node("Relu", ["s"], "z")
    elif post == "clip":
        b.const("lo", np.float32(0.0))
        b.const("hi", np.float32(1.5))
        b.node("Clip", ["s", "lo", "hi"], "z")
    else:
        b.node("Identity", ["s"], "z")
    b.output("z")
    feeds = {"x": rng.standard_normal((2, 32, 10, 10)).astype(np.float32),
             "r": rng.standard_normal((2, 48, 10, 10)).astype(np.float32)}
    return b.graph(), feeds


@pytest.mark.parametrize("mode", ["implicit", "im2col"])
@pytest.mark.parametrize("sk", [1, 3, "stream"])
@pytest.mark.parametrize("post,res_first", [("relu", False), ("relu", True), ("clip", False),
                                            ("none", True)])
def test_conv_residual_epilogue(post, res_first, sk, mode, hip_ctx):
    """A residual add (+ Relu / Clip / nothing) folded into the conv epilogue
    (or the split-K reduce, or the stream-K fix-up) matches the oracle and
    equals the unfused device result bit for bit."""
    sched = (MfmaSchedule(64, 64, 16, 2, 2, 32, True).with_stream_k() if sk == "stream"
             else MfmaSchedule(64, 64, 16, 2, 2, 32, True, sk))
    g, feeds = _conv_residual_graph(post, res_first)
    c, got, want = device_run(g, feeds, conv_mode=mode, ctx=hip_ctx,
                              schedule_fn=lambda n, mnk: sched, winograd=False)
    assert sum(1 for n in c.graph.nodes if n.attrs.get("residual_subgraph")) == 1
    assert "elementwise" not in {l.kind for l in c.module.plan}
    assert_close("z", got["z"], want["z"])
    g2, _ = _conv_residual_graph(post, res_first)
    c2, got2, _ = device_run(g2, feeds, conv_mode=mode, ctx=hip_ctx,
                             schedule_fn=lambda n, mnk: sched, fuse_residual=False, winograd=False)
    assert not any(n.attrs.get("residual_subgraph") for n in c2.graph.nodes)
    np.testing.assert_array_equal(got["z"], got2["z"])


@pytest.mark.parametrize("mode", ["implicit", "im2col"])
@pytest.mark.parametrize("case", [(2, 16, 14, 14, 32, 3, 1, 1), (5, 16, 64, 64, 64, 3, 1, 1),
                                  (1, 64, 7, 7, 128, 3, 1, 1), (3, 24, 33, 33, 40, 3, 2, 1)],
                         ids=lambda c: "x".join(map(str, c)))
def test_conv_stream_k(case, mode, hip_ctx):
    """Stream-K: with fewer tiles than CUs every tile is assembled from
    pieces (some one K step long); with 320 tiles the first 256 are done whole
    and the other 64 in pieces. Correct on the first run and on a repeat with
    another input in between (the workspace is rewritten every run), and the
    same bits every time (pieces are added in K order)."""
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor
    from mdlc_amd.compiler import compile_graph
    from oracle.reference import run_reference

    sched = MfmaSchedule(64, 64, 16, 2, 2, 32, True).with_stream_k()
    g, feeds = _conv_graph(*case)
    c = compile_graph(g, feeds=feeds, conv_mode=mode, schedule_fn=lambda n, mnk: sched,
                      winograd=False)
    kinds = [l.kind for l in c.module.plan]
    assert kinds[-1] == "streamk_fixup"
    main = c.module.plan[-2]
    assert main.meta["stream_k"] and main.grid[0] == main.meta["ksplit"] + 256
    ex = HipExecutor(c.module, hip_ctx)
    try:
        y1 = ex.run(feeds)["outputs"]["y"]
        ex.run({"x": (feeds["x"][::-1] * 0.5).copy()})
        y2 = ex.run(feeds)["outputs"]["y"]
    finally:
        ex.close()
    want = run_reference(c.graph, feeds)["y"]
    assert_close("y", y1, want)
    np.testing.assert_array_equal(y1, y2)


@pytest.mark.parametrize("case", [(2, 16, 16, 16, 32, 3, 1, 1), (1, 64, 14, 14, 128, 3, 1, 1)],
                         ids=lambda c: "x".join(map(str, c)))
def test_splitk_reduce_vector_and_scalar_forms_agree(case, hip_ctx, monkeypatch):
    """The split-K reduce with four outputs per thread (here hw = 256, 196)
    and with one give the same bits, and match the oracle."""
    from mdlc_amd.codegen.hip import emit

    sched = MfmaSchedule(64, 64, 16, 2, 2, 32, True, 5)
    g, feeds = _conv_graph(*case)
    c, got, want = device_run(g, feeds, ctx=hip_ctx, schedule_fn=lambda n, mnk: sched,
                              winograd=False)
    (red,) = [l for l in c.module.plan if l.kind == "splitk_reduce"]
    assert red.kernel_name.startswith("splitk_reduce4_")
    assert_close("y", got["y"], want["y"])
    monkeypatch.setattr(emit, "REDUCE_VEC", 1)
    g2, _ = _conv_graph(*case)
    c2, got2, _ = device_run(g2, feeds, ctx=hip_ctx, schedule_fn=lambda n, mnk: sched,
                             winograd=False)
    assert not any(l.kernel_name.startswith("splitk_reduce4_") for l in c2.module.plan)
    np.testing.assert_array_equal(got["y"], got2["y"])


@pytest.mark.parametrize("n", [1, 2, 8])
def test_conv_no_bias_no_act(n, hip_ctx):
    g, feeds = _conv_graph(n, 5, 11, 11, 6, 3, 1, 1, act=None, bias=False, seed=4)
    _, got, want = device_run(g, feeds, ctx=hip_ctx)
    assert_close("y", got["y"], want["y"])


def test_im2col_kernel_is_bitwise(hip_ctx):
    """The column matrix equals the oracle's im2col bit for bit (reference
    tests/test_codegen_kernels.py:57-74, seed 1, C,H,W = 3,9,9, k3 s1 p1),
    here at batch 2 with the batched column order p = (n, oh, ow)."""
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor
    from mdlc_amd.compiler import compile_graph
    from oracle import ops

    g, feeds = _conv_graph(2, 3, 9, 9, 8, 3, 1, 1, seed=1)
    c = compile_graph(g, feeds=feeds, conv_mode="im2col")
    ex = HipExecutor(c.module, hip_ctx)
    try:
        ex.run(feeds)
        cols_name = next(iter(c.module.scratch_shapes))
        dev = ex.read(cols_name)
    finally:
        ex.close()
    ref, oh, ow = ops.im2col(feeds["x"], 3, 3, 1, 1, 1, 1, ((1, 1), (1, 1)))
    ref = ref.transpose(1, 0, 2).reshape(27, 2 * oh * ow)          # [K, N*OH*OW]
    P = ref.shape[1]
    np.testing.assert_allclose(dev[:, :P], ref, rtol=BITWISE.rtol, atol=BITWISE.atol)
    assert np.all(dev[:, P:] == 0)


@pytest.mark.parametrize("n", [1, 3])
@pytest.mark.parametrize("act", ["Relu", "Clip", None])
def test_depthwise_conv(n, act, hip_ctx):
    for (c, h, k, s) in [(16, 12, 3, 1), (32, 13, 3, 2)]:
        g, feeds = _conv_graph(n, c, h, h, c, k, s, 1, act=act, group=c, seed=6)
        _, got, want = device_run(g, feeds, ctx=hip_ctx)
        assert_close("y", got["y"], want["y"])


@pytest.mark.parametrize("N", [256, 1001, 4, 3])
def test_elementwise_chain(N, hip_ctx):
    """y = relu(a + b) * c (reference test_codegen_kernels.py:101-120, seed 3)."""
    rng = np.random.default_rng(3)
    b = GraphBuilder("ew")
    for nm in "abc":
        b.input(nm, (N,))
    b.node("Add", ["a", "b"], "s")
    b.node("Relu", ["s"], "r")
    b.node("Mul", ["r", "c"], "y")
    b.output("y")
    feeds = {nm: rng.standard_normal(N).astype(np.float32) for nm in "abc"}
    c, got, want = device_run(b.graph(), feeds, ctx=hip_ctx)
    fe = [n for n in c.graph.nodes if n.op_type == "FusedElementwise"]
    assert len(fe) == 1
    assert_close("y", got["y"], want["y"])


def test_elementwise_all_activations(hip_ctx):
    """Each activation and binary op as its own group (single pointwise
    nodes are lowered as one-member groups), all reading one input, plus one
    long fused chain."""
    rng = np.random.default_rng(9)
    N = 4099
    b = GraphBuilder("acts")
    b.input("x", (N,))
    b.input("z", (N,))
    b.const("two", np.float32(2.0))
    singles = [("Relu", {}), ("Sigmoid", {}), ("Tanh", {}), ("LeakyRelu", {"alpha": 0.1}),
               ("HardSwish", {}), ("HardSigmoid", {"alpha": 0.25, "beta": 0.4})]
    for i, (op, attrs) in enumerate(singles):
        b.output(b.node(op, ["x"], f"s{i}", **attrs))
    for op in ("Add", "Sub", "Mul", "Div"):
        b.output(b.node(op, ["x", "z"], f"b_{op}"))
    cur = "x"
    for i, op in enumerate(["Sigmoid", "Mul", "Sub", "Tanh", "HardSwish"]):
        cur = b.node(op, [cur, "two"] if op in ("Mul", "Sub") else [cur], f"c{i}")
    b.output(cur)
    feeds = {"x": (rng.standard_normal(N) * 3).astype(np.float32),
             "z": (rng.uniform(0.5, 2.0, N) * np.sign(rng.standard_normal(N))).astype(np.float32)}
    c, got, want = device_run(b.graph(), feeds, ctx=hip_ctx)
    assert c.module.fallbacks() == []
    for name in got:
        assert_close(name, got[name], want[name])


@pytest.mark.parametrize("n", [1, 4])
def test_maxpool_and_gap(n, hip_ctx):
    rng = np.random.default_rng(11)
    b = GraphBuilder("pool")
    b.input("x", (n, 8, 17, 17))
    b.node("MaxPool", ["x"], "m", kernel_shape=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1])
    b.node("GlobalAveragePool", ["m"], "gp")
    b.node("Flatten", ["gp"], "y", axis=1)
    b.output("y")
    b.output("m")
    feeds = {"x": rng.standard_normal((n, 8, 17, 17)).astype(np.float32)}
    _, got, want = device_run(b.graph(), feeds, ctx=hip_ctx)
    assert_close("m", got["m"], want["m"], BITWISE)
    assert_close("y", got["y"], want["y"], DEVICE_TENSOR)


@pytest.mark.parametrize("win", [(3, 3, 1, 1, 1, 1, 1, 0), (3, 3, 2, 2, 1, 1, 1, 0),
                                 (2, 2, 2, 2, 0, 0, 1, 0), (3, 2, 1, 3, 1, 0, 1, 0),
                                 (3, 3, 2, 2, 1, 1, 2, 0), (3, 3, 2, 2, 0, 0, 1, 1)],
                         ids=lambda w: "k{}x{}_s{}x{}_p{}{}_d{}_c{}".format(*w))
def test_maxpool_windows(win, hip_ctx):
    """Windows, strides (adjacent outputs per thread 4, 2 and 1), padding,
    dilation and ceil mode over widths that are not multiples of the per-thread
    output count; max pooling is exact, so the match is bitwise."""
    kh, kw, sh, sw, ph, pw, d, ceil = win
    rng = np.random.default_rng(12)
    b = GraphBuilder("mp")
    b.input("x", (2, 3, 15, 13))
    b.node("MaxPool", ["x"], "m", kernel_shape=[kh, kw], strides=[sh, sw], pads=[ph, pw, ph, pw],
           dilations=[d, d], ceil_mode=ceil)
    b.output("m")
    # (the ceil-mode case divides evenly: the oracle's strided slice cannot
    # express a partial last window, ops.py:119-124)
    feeds = {"x": rng.standard_normal((2, 3, 15, 13)).astype(np.float32)}
    _, got, want = device_run(b.graph(), feeds, ctx=hip_ctx)
    assert_close("m", got["m"], want["m"], BITWISE)


def test_fused_elementwise_dedup_shares_kernel():
    """Structurally identical groups compile to one kernel (CPU-side check
    that still belongs with the kernel tests)."""
    from mdlc_amd.compiler import compile_graph
    from mdlc_amd.tools.build_resnet18 import build_resnet18

    c = compile_graph(build_resnet18(batch=1), fuse_residual=False)
    ew = {l.kernel_name for l in c.module.plan if l.kind == "elementwise"}
    assert len(ew) == 1
    assert isinstance(Node, type)
