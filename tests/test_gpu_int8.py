"""INT8 path on the device: every int8 code and int32-derived output is
bit-exact against the oracle's build-defined semantics (oracle/quant.py).

The reference has no quantized operator, so these are the only parity
checks for this row; the oracle's own semantics are pinned on the CPU in
tests/test_oracle.py (integer closed forms, float64 route, round-half-even).
"""

from __future__ import annotations

import numpy as np
import pytest

from gpu_util import assert_close, device_run
import mdlc_amd.codegen.hip.emit_int8 as emit_int8
import mdlc_amd.codegen.schedule as S
from mdlc_amd.codegen.schedule import MfmaSchedule
from mdlc_amd.tools.build_repvit_int8 import build_repvit_int8, gelu_table, make_input
from mdlc_amd.tools.graph_builder import GraphBuilder

pytestmark = pytest.mark.gpu


def _qconv_graph(n, c, h, w, oc, k, s, *, group=1, relu=False, seed=0, scale_in=0.05):
    rng = np.random.default_rng(seed)
    b = GraphBuilder("qc")
    b.input("x", (n, c, h, w))
    b.node("QuantizeLinear", ["x"], "xq", inv_scale=float(np.float32(1 / scale_in)))
    icg = c // group
    b.const("w", rng.integers(-127, 128, (oc, icg, k, k)).astype(np.int8))
    b.const("b", rng.integers(-3000, 3000, oc).astype(np.int32))
    b.const("m", rng.uniform(0.0005, 0.004, oc).astype(np.float32))
    p = (k - 1) // 2
    attrs = dict(kernel_shape=[k, k], strides=[s, s], pads=[p] * 4, group=group)
    if relu:
        attrs["activation"] = "Relu"
    b.node("QConv", ["xq", "w", "b", "m"], "y", **attrs)
    b.output("y")
    b.output("xq")
    x = (rng.standard_normal((n, c, h, w)) * 3).astype(np.float32)
    return b.graph(), {"x": x}


QCONV_CASES = [
    # n, c, h, w, oc, k, s, group
    (2, 48, 14, 14, 96, 1, 1, 1),        # pointwise: dense GEMM over NHWC
    (1, 96, 9, 9, 48, 1, 1, 1),
    (2, 32, 12, 12, 64, 3, 1, 1),        # tap-major gather, C % 16 == 0
    (2, 32, 13, 13, 48, 3, 2, 1),
    (2, 3, 30, 30, 24, 3, 2, 1),         # byte gather, C = 3
    (2, 24, 15, 15, 48, 3, 2, 1),        # byte gather, C = 24
    (2, 48, 14, 14, 48, 3, 1, 48),       # depthwise, 16-channel vectors
    (2, 48, 15, 15, 48, 3, 2, 48),
    (1, 24, 10, 10, 24, 3, 1, 24),       # depthwise, scalar channels
]


@pytest.mark.parametrize("relu", [False, True])
@pytest.mark.parametrize("case", QCONV_CASES, ids=lambda c: "x".join(map(str, c)))
def test_qconv_bit_exact(case, relu, hip_ctx):
    n, c, h, w, oc, k, s, group = case
    g, feeds = _qconv_graph(n, c, h, w, oc, k, s, group=group, relu=relu)
    cmod, got, want = device_run(g, feeds, ctx=hip_ctx)
    assert cmod.module.fallbacks() == []
    assert got["xq"].dtype == np.int8 and got["y"].dtype == np.int8
    np.testing.assert_array_equal(got["xq"], want["xq"])
    np.testing.assert_array_equal(got["y"], want["y"])
    v = want["y"].astype(int)
    assert v.std() > 3 and np.mean(np.abs(v) == 127) < 0.5        # non-degenerate


@pytest.mark.parametrize("impl", ["mfma", "vector"])
@pytest.mark.parametrize("case", [(2, 48, 14, 14, 3, 1), (2, 48, 15, 15, 3, 2), (1, 64, 9, 9, 5, 1),
                                  (3, 32, 8, 8, 3, 2), (1, 384, 7, 7, 3, 1)],
                         ids=lambda c: "x".join(map(str, c)))
def test_qdepthwise_matrix_core_and_vector_paths(case, impl, hip_ctx):
    """Depthwise int8 convs (C % 16 == 0) as block-diagonal MFMA GEMMs and on
    the vector kernel: both bit-exact (5x5 window: 25 taps, K padded to 448)."""
    n, c, h, w, k, s = case
    g, feeds = _qconv_graph(n, c, h, w, c, k, s, group=c, relu=True, seed=7)
    cmod, got, want = device_run(g, feeds, ctx=hip_ctx, int8_depthwise=impl)
    kinds = [l.kind for l in cmod.module.plan]
    assert ("qdwconv" in kinds) == (impl == "vector")
    np.testing.assert_array_equal(got["y"], want["y"])


class _Fixed:
    """A schedule source that returns one schedule for every problem."""

    def __init__(self, sched):
        self.sched = sched

    def schedule_problem(self, problem):
        return self.sched


QSCHEDULES = [MfmaSchedule(256, 256, 128, 4, 2, 32, True),   # two register sets in flight
              MfmaSchedule(256, 256, 64, 2, 2, 32, True),    # 256 accumulators, one set
              MfmaSchedule(128, 64, 128, 2, 1, 16, True),
              MfmaSchedule(32, 32, 64, 1, 1, 32, True),
              MfmaSchedule(128, 128, 256, 2, 2, 16, False),  # single LDS buffer, 256-byte K tiles
              MfmaSchedule(256, 256, 128, 2, 2, 32, True, 1, False, 2),   # interleaved pipeline
              MfmaSchedule(128, 64, 64, 2, 2, 16, True, 1, False, 2),
              MfmaSchedule(256, 256, 128, 4, 4, 16, True)]     # 16 waves


@pytest.mark.parametrize("sched", QSCHEDULES, ids=lambda s: s.key())
@pytest.mark.parametrize("case", [(2, 3, 17, 17, 24, 3, 2), (2, 6, 11, 11, 40, 3, 1),
                                  (2, 12, 11, 11, 24, 3, 2), (2, 24, 9, 9, 48, 3, 1),
                                  (2, 48, 9, 9, 72, 3, 2), (2, 64, 7, 7, 264, 1, 1)],
                         ids=lambda c: "x".join(map(str, c)))
def test_qconv_gather_widths_and_tiles(case, sched, hip_ctx):
    """Gather widths 1/2/4/8/16 bytes (C = 3, 6, 12, 24, 48) and a dense
    pointwise conv whose N is not a tile multiple, under tiles from 32x32 to
    256x256 (ragged M, N and K everywhere)."""
    g, feeds = _qconv_graph(*case, relu=True, seed=4)
    cmod, got, want = device_run(g, feeds, ctx=hip_ctx, schedule_fn=_Fixed(sched))
    (launch,) = [l for l in cmod.module.plan if l.kind == "qgemm"]
    assert launch.meta["sched"] == sched
    np.testing.assert_array_equal(got["y"], want["y"])


@pytest.mark.parametrize("sched", [None, MfmaSchedule(64, 64, 128, 2, 2, 16, True),
                                   MfmaSchedule(128, 128, 64, 2, 2, 32, True),
                                   MfmaSchedule(32, 64, 64, 1, 2, 32, True)] + QSCHEDULES[:2],
                         ids=lambda s: "default" if s is None else s.key())
@pytest.mark.parametrize("out", ["int8", "float32", "int32"])
def test_qgemm_bit_exact(sched, out, hip_ctx):
    rng = np.random.default_rng(3)
    M, N, K = 77, 130, 384
    b = GraphBuilder("qg")
    b.input("x", (M, K))
    b.node("QuantizeLinear", ["x"], "xq", inv_scale=20.0)
    b.const("w", rng.integers(-127, 128, (N, K)).astype(np.int8))
    b.const("b", rng.integers(-20000, 20000, N).astype(np.int32))
    b.const("m", rng.uniform(1e-4, 1e-3, N).astype(np.float32))
    b.node("QGemm", ["xq", "w", "b", "m"], "y", transB=1, out_dtype=out)
    b.output("y")
    feeds = {"x": rng.standard_normal((M, K)).astype(np.float32)}
    _, got, want = device_run(b.graph(), feeds, ctx=hip_ctx,
                              schedule_fn=None if sched is None else _Fixed(sched))
    assert got["y"].dtype == want["y"].dtype
    np.testing.assert_array_equal(got["y"], want["y"])


@pytest.mark.parametrize("c", [32, 192])
def test_qadd_qlut_qgap(c, hip_ctx):
    """Add, lookup and the pool, bit-exact; C = 192 spreads each image's pool
    over three 64-channel workgroups."""
    rng = np.random.default_rng(5)
    b = GraphBuilder("q")
    b.input("x", (2, c, 7, 7))
    b.input("z", (2, c, 7, 7))
    b.node("QuantizeLinear", ["x"], "xq", inv_scale=10.0)
    b.node("QuantizeLinear", ["z"], "zq", inv_scale=30.0)
    b.node("QAdd", ["xq", "zq"], "s", ma=0.75, mb=0.5)
    b.const("t", gelu_table(0.1, 0.05))
    b.node("QLut", ["s", "t"], "l")
    b.node("QGlobalAveragePool", ["l"], "p", mult=float(np.float32(1 / 49)))
    b.node("Flatten", ["p"], "f", axis=1)
    for o in ("s", "l", "f"):
        b.output(o)
    feeds = {"x": (rng.standard_normal((2, c, 7, 7)) * 5).astype(np.float32),
             "z": (rng.standard_normal((2, c, 7, 7)) * 5).astype(np.float32)}
    cm, got, want = device_run(b.graph(), feeds, ctx=hip_ctx, all_tensors=True)
    (gap,) = [l for l in cm.module.plan if l.kind == "qgap"]
    assert gap.grid[1] == (c // 64 if c % 64 == 0 else 1)
    for name in want:
        if name in got:
            np.testing.assert_array_equal(got[name], want[name], err_msg=name)
    assert np.mean(np.abs(got["s"].astype(int)) == 127) > 0.01          # clamp path exercised


@pytest.mark.parametrize("mode", ["mlp", "epilogues", "unfused"])
@pytest.mark.parametrize("batch", [1, 2, 32])
def test_repvit_int8_every_tensor_bit_exact(batch, mode, hip_ctx):
    """Every int8 tensor the module materializes, and the logits, equal the
    oracle's — with the channel mixers as fused MLP launches, with the GELU
    lookups and residual adds folded into the conv epilogues, and with
    neither (separate lookup/add launches, vector depthwise kernel)."""
    g = build_repvit_int8(batch=batch)
    feeds = {"input": make_input(batch)}
    c, got, want = device_run(g, feeds, ctx=hip_ctx, all_tensors=True,
                              fuse_int8_epilogues=mode != "unfused", fuse_int8_mlp=mode == "mlp",
                              int8_depthwise="vector" if mode == "unfused" else "mfma")
    assert c.module.fallbacks() == []
    nq = sum(l.kind == "qmlp" for l in c.module.plan)
    assert nq == (21 if mode == "mlp" else 0)
    nf = sum(l.kind == "qconv_first" for l in c.module.plan)     # stem + its GELU + the quantize
    assert nf == (0 if mode == "unfused" else 1)
    epis = [l.meta.get("epilogue", 0) for l in c.module.plan if l.kind == "qgemm"]
    want_epis = (0, 0) if mode == "unfused" else (24 - nq - nf, 23 - nq)
    assert (epis.count(1), epis.count(2)) == want_epis
    n = 0
    for name, v in got.items():
        w = want[name]
        if w.dtype == np.int8:
            np.testing.assert_array_equal(v, w, err_msg=name)
            n += 1
    assert n >= {"mlp": 30, "epilogues": 70, "unfused": 120}[mode]
    np.testing.assert_array_equal(got["logits"], want["logits"])


def _mlp_graph(n, c, e, hw, *, relu1=False, relu2=False, seed=3, mixer=0, relu_dw=False):
    """Quantize -> 1x1 QConv c->e -> QLut -> 1x1 QConv e->c -> QAdd(xq, .):
    a RepViT channel mixer with random weights, table and multipliers sized
    to keep the codes away from the clamps. ``mixer`` = k puts a depthwise
    kxk stride-1 QConv (the token mixer) in front: xq is then its output."""
    rng = np.random.default_rng(seed)
    b = GraphBuilder("mlp")
    b.input("x", (n, c, hw, hw))
    if mixer:
        b.node("QuantizeLinear", ["x"], "z", inv_scale=20.0)
        b.const("wd", rng.integers(-127, 128, (c, 1, mixer, mixer)).astype(np.int8))
        b.const("bd", rng.integers(-2000, 2000, c).astype(np.int32))
        b.const("md", (rng.uniform(0.5, 1.5, c) * 0.01 / mixer).astype(np.float32))
        p = mixer // 2
        b.node("QConv", ["z", "wd", "bd", "md"], "xq", kernel_shape=[mixer, mixer], strides=[1, 1],
               pads=[p] * 4, group=c, **({"activation": "Relu"} if relu_dw else {}))
    else:
        b.node("QuantizeLinear", ["x"], "xq", inv_scale=20.0)
    b.const("w1", rng.integers(-127, 128, (e, c, 1, 1)).astype(np.int8))
    b.const("b1", rng.integers(-3000, 3000, e).astype(np.int32))
    b.const("m1", (rng.uniform(0.5, 1.5, e) * 0.01 / np.sqrt(c)).astype(np.float32))
    b.const("t", rng.integers(-127, 128, 256).astype(np.int8))
    b.const("w2", rng.integers(-127, 128, (c, e, 1, 1)).astype(np.int8))
    b.const("b2", rng.integers(-3000, 3000, c).astype(np.int32))
    b.const("m2", (rng.uniform(0.5, 1.5, c) * 0.0075 / np.sqrt(e)).astype(np.float32))
    one = dict(kernel_shape=[1, 1], strides=[1, 1], pads=[0] * 4)
    b.node("QConv", ["xq", "w1", "b1", "m1"], "h0", **one, **({"activation": "Relu"} if relu1 else {}))
    b.node("QLut", ["h0", "t"], "h")
    b.node("QConv", ["h", "w2", "b2", "m2"], "y0", **one, **({"activation": "Relu"} if relu2 else {}))
    b.node("QAdd", ["xq", "y0"], "y", ma=0.6, mb=0.35)
    b.output("y")
    return b.graph(), {"x": (rng.standard_normal((n, c, hw, hw)) * 3).astype(np.float32)}


class _MlpRows:
    """A schedule source that forces the fused MLP kernel's rows per workgroup."""

    def __init__(self, bm):
        self.bm = bm

    def qmlp_layout(self, C, E, M):
        from mdlc_amd.codegen.schedule import qmlp_layout
        return qmlp_layout(C, E, M, bm=self.bm)

    def __call__(self, node, mnk):
        from mdlc_amd.codegen.schedule import default_qschedule
        return default_qschedule(*mnk)


@pytest.mark.parametrize("bm", [None, 16, 32, 64])
@pytest.mark.parametrize("case", [(2, 48, 96, 14, False, False), (2, 96, 192, 9, False, False),
                                  (1, 192, 384, 7, False, False), (2, 384, 768, 7, False, False),
                                  (1, 32, 64, 5, True, False), (3, 48, 160, 5, False, True),
                                  (2, 64, 128, 6, True, True)],
                         ids=lambda c: "n{}c{}e{}hw{}{}{}".format(*c[:4], "_relu1" if c[4] else "",
                                                               "_relu2" if c[5] else ""))
def test_qmlp_bit_exact(case, bm, hip_ctx):
    """The fused channel mixer equals the oracle and the two-conv launches it
    replaces bit for bit: RepViT's four stage widths, K padding on either
    GEMM (C = 32, E = 160), ReLU clamps, row tails, each row tiling."""
    from mdlc_amd.codegen.schedule import qmlp_layout

    n, c, e, hw, r1, r2 = case
    if bm is not None and qmlp_layout(c, e, n * hw * hw, bm=bm) is None:
        pytest.skip(f"no {bm}-row tiling for C={c}, E={e}")
    g, feeds = _mlp_graph(n, c, e, hw, relu1=r1, relu2=r2)
    fn = None if bm is None else _MlpRows(bm)
    cmod, got, want = device_run(g, feeds, ctx=hip_ctx, schedule_fn=fn, fuse_int8_mlp="always")
    assert [l.kind for l in cmod.module.plan] == ["quantize", "qmlp"]
    np.testing.assert_array_equal(got["y"], want["y"])
    v = want["y"].astype(int)
    assert v.std() > 3 and np.mean(np.abs(v) == 127) < 0.5
    g2, _ = _mlp_graph(n, c, e, hw, relu1=r1, relu2=r2)
    _, got2, _ = device_run(g2, feeds, ctx=hip_ctx, fuse_int8_mlp=False)
    np.testing.assert_array_equal(got["y"], got2["y"])


@pytest.mark.parametrize("case", [(2, 48, 96, 14, 3, False), (2, 96, 192, 9, 3, False),
                                  (1, 192, 384, 7, 3, True), (3, 64, 128, 5, 3, False),
                                  (1, 32, 64, 7, 5, True), (2, 16, 32, 4, 3, False)],
                         ids=lambda c: "n{}c{}e{}hw{}k{}{}".format(*c[:5], "_relu" if c[5] else ""))
@pytest.mark.parametrize("weights", ["regs", "lds"])
def test_qmlp_token_mixer_bit_exact(case, weights, hip_ctx, monkeypatch):
    """The depthwise token mixer computed in the fused kernel's prologue:
    image borders (3x3 and 5x5 windows), row tails that cross images, and a
    ReLU clamp — against the oracle and against the separate launches, with
    the mixer's weights in registers (these grids fit one workgroup per CU)
    and in LDS (the form of grids larger than the chip, forced here)."""
    import mdlc_amd.codegen.hip.emit_int8 as emit_int8

    n, c, e, hw, k, relu = case
    if weights == "lds":
        form = emit_int8.qmlp_latency_form
        monkeypatch.setattr(emit_int8, "qmlp_latency_form", lambda *a: form(*a)[:2] + (False,))
    g, feeds = _mlp_graph(n, c, e, hw, mixer=k, relu_dw=relu, seed=9)
    cmod, got, want = device_run(g, feeds, ctx=hip_ctx, fuse_int8_mlp="always")
    assert [l.kind for l in cmod.module.plan] == ["quantize", "qmlp"]
    assert cmod.module.plan[1].meta["mixer"]
    assert ("_wr_" in cmod.module.plan[1].kernel_name) == (weights == "regs")
    np.testing.assert_array_equal(got["y"], want["y"])
    v = want["y"].astype(int)
    assert v.std() > 3 and np.mean(np.abs(v) == 127) < 0.5
    g2, _ = _mlp_graph(n, c, e, hw, mixer=k, relu_dw=relu, seed=9)
    _, got2, _ = device_run(g2, feeds, ctx=hip_ctx, fuse_int8_epilogues=False)
    np.testing.assert_array_equal(got["y"], got2["y"])


def _qconv_epilogue_graph(n, c, hw, oc, k, epilogue, *, res_first, seed=5):
    """QConv (3x3 gather or 1x1 dense) followed by a QLut or by a QAdd with a
    second int8 tensor of the conv output's shape."""
    rng = np.random.default_rng(seed)
    b = GraphBuilder("qe")
    b.input("x", (n, c, hw, hw))
    b.input("r", (n, oc, hw, hw))
    b.node("QuantizeLinear", ["x"], "xq", inv_scale=20.0)
    b.node("QuantizeLinear", ["r"], "rq", inv_scale=25.0)
    b.const("w", rng.integers(-127, 128, (oc, c, k, k)).astype(np.int8))
    b.const("b", rng.integers(-3000, 3000, oc).astype(np.int32))
    b.const("m", rng.uniform(0.0005, 0.004, oc).astype(np.float32))
    p = (k - 1) // 2
    b.node("QConv", ["xq", "w", "b", "m"], "y", kernel_shape=[k, k], strides=[1, 1], pads=[p] * 4)
    if epilogue == "lut":
        b.const("t", rng.integers(-127, 128, 256).astype(np.int8))
        b.node("QLut", ["y", "t"], "z")
    else:
        ins = ["rq", "y"] if res_first else ["y", "rq"]
        b.node("QAdd", ins, "z", ma=0.7, mb=0.45)
    b.output("z")
    feeds = {"x": (rng.standard_normal((n, c, hw, hw)) * 3).astype(np.float32),
             "r": (rng.standard_normal((n, oc, hw, hw)) * 3).astype(np.float32)}
    return b.graph(), feeds


@pytest.mark.parametrize("sched", [None] + QSCHEDULES[:1] + QSCHEDULES[2:],
                         ids=lambda s: "default" if s is None else s.key())
@pytest.mark.parametrize("case", [("lut", 1, False), ("lut", 3, False), ("add", 1, False),
                                  ("add", 1, True), ("add", 3, True)],
                         ids=lambda c: f"{c[0]}_k{c[1]}{'_resfirst' if c[2] else ''}")
@pytest.mark.parametrize("oc", [48, 30])
def test_qconv_fused_epilogues(case, oc, sched, hip_ctx):
    """The fused lookup and residual add equal the unfused ops bit for bit,
    for either QAdd operand order, an output width that is not a multiple of
    four (byte stores) and several tiles."""
    epilogue, k, res_first = case
    g, feeds = _qconv_epilogue_graph(2, 32, 9, oc, k, epilogue, res_first=res_first)
    fn = None if sched is None else _Fixed(sched)
    cmod, got, want = device_run(g, feeds, ctx=hip_ctx, schedule_fn=fn)
    assert [n.op_type for n in cmod.graph.nodes].count("QConv") == 1
    assert len(cmod.graph.nodes) == (2 if epilogue == "lut" else 3)    # quantize(s) + fused conv
    np.testing.assert_array_equal(got["z"], want["z"])
    g2, _ = _qconv_epilogue_graph(2, 32, 9, oc, k, epilogue, res_first=res_first)
    _, got2, _ = device_run(g2, feeds, ctx=hip_ctx, schedule_fn=fn, fuse_int8_epilogues=False)
    np.testing.assert_array_equal(got["z"], got2["z"])


@pytest.mark.parametrize("sched", [None, QSCHEDULES[0], QSCHEDULES[5], QSCHEDULES[7]],
                         ids=lambda s: "default" if s is None else s.key())
def test_qgemm_int32_accumulators_exact(sched, hip_ctx):
    """The raw int32 accumulators (out_dtype int32: acc + bias, no requant)
    at K = 4096, with rows and columns of +-127 codes so that |acc| reaches
    127 * 127 * 4096 = 66e6 > 2^24 (where a float32 route would round),
    equal the exact int64 product."""
    rng = np.random.default_rng(21)
    M, N, K = 300, 260, 4096
    x = rng.integers(-127, 128, (M, K)).astype(np.int8)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    x[:3] = 127
    x[3] = -127
    w[:2] = 127
    w[5] = -127
    bias = rng.integers(-2 ** 20, 2 ** 20, N).astype(np.int32)
    b = GraphBuilder("qacc")
    b.input("xq", (M, K), dtype="int8")
    b.const("w", w)
    b.const("b", bias)
    b.const("m", np.ones(N, np.float32))
    b.node("QGemm", ["xq", "w", "b", "m"], "y", transB=1, out_dtype="int32")
    b.output("y")
    _, got, want = device_run(b.graph(), {"xq": x}, ctx=hip_ctx,
                              schedule_fn=None if sched is None else _Fixed(sched))
    exact = x.astype(np.int64) @ w.astype(np.int64).T + bias
    assert got["y"].dtype == np.int32 and np.abs(exact).max() > 2 ** 24
    np.testing.assert_array_equal(want["y"], exact)
    np.testing.assert_array_equal(got["y"], exact)


def test_int8_gemm_4096_cube_rows_exact(hip_ctx):
    """The compute-bound int8 shape (M = N = K = 4096) with the shipped
    schedule: every output against an exact float64 product (|acc| < 2^53)."""
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor
    from mdlc_amd.compiler import compile_graph

    rng = np.random.default_rng(11)
    M = N = K = 4096
    b = GraphBuilder("q4k")
    b.input("xq", (M, K), dtype="int8")
    wq = rng.integers(-127, 128, (N, K)).astype(np.int8)
    bias = rng.integers(-10000, 10000, N).astype(np.int32)
    mult = rng.uniform(2e-6, 1e-5, N).astype(np.float32)
    b.const("w", wq)
    b.const("b", bias)
    b.const("m", mult)
    b.node("QGemm", ["xq", "w", "b", "m"], "y", transB=1)
    b.output("y")
    xq = rng.integers(-127, 128, (M, K)).astype(np.int8)
    c = compile_graph(b.graph(), feeds={"xq": xq})
    ex = HipExecutor(c.module, hip_ctx)
    try:
        y = ex.run({"xq": xq})["outputs"]["y"]
    finally:
        ex.close()
    for r0 in range(0, M, 1024):                   # all rows, 1024 at a time
        acc = (xq[r0:r0 + 1024].astype(np.float64) @ wq.T.astype(np.float64)).astype(np.int64) + bias
        f = acc.astype(np.int32).astype(np.float32) * mult
        want = np.clip(np.rint(f), -127, 127).astype(np.int8)
        np.testing.assert_array_equal(y[r0:r0 + 1024], want)


@pytest.mark.parametrize("case", [(2, 3, 31, 24, 3, 2, "lut"), (1, 3, 16, 24, 3, 2, None),
                                  (2, 1, 9, 8, 5, 1, "lut"), (1, 4, 12, 16, 3, 1, "relu"),
                                  (3, 2, 7, 12, 3, 2, None), (1, 3, 20, 36, 3, 2, "lut")],
                         ids=lambda c: "n{}c{}hw{}oc{}k{}s{}_{}".format(*c))
@pytest.mark.parametrize("cus,cap", [(256, None), (2, None), (2, 3)], ids=["bands1", "bandsR", "loop"])
def test_first_conv_quantizes_its_input(case, cus, cap, hip_ctx, monkeypatch):
    """QuantizeLinear folded into a small first QConv (float NCHW in, bands of
    output rows quantized into LDS once, 16x16x64 int8 MFMAs over (tap,
    channel)), with a fused lookup, a ReLU or neither, single-row and
    several-row bands (a partial last band included): equal to the oracle
    and to the separate quantize + conv launches."""
    n, c, hw, oc, k, s, post = case
    monkeypatch.setattr(S, "CUS", cus)      # few CUs: the shapes take bands of several rows
    if cap:                                 # three workgroups taking the bands in turn
        monkeypatch.setattr(emit_int8, "qconv_first_grid", lambda: cap)

    def graph():
        rng = np.random.default_rng(21)
        b = GraphBuilder("first")
        b.input("x", (n, c, hw, hw))
        b.node("QuantizeLinear", ["x"], "xq", inv_scale=25.0)
        b.const("w", rng.integers(-127, 128, (oc, c, k, k)).astype(np.int8))
        b.const("b", rng.integers(-3000, 3000, oc).astype(np.int32))
        b.const("m", (rng.uniform(0.5, 1.5, oc) * 0.01 / np.sqrt(c * k * k)).astype(np.float32))
        attrs = dict(kernel_shape=[k, k], strides=[s, s], pads=[k // 2] * 4)
        if post == "relu":
            attrs["activation"] = "Relu"
        b.node("QConv", ["xq", "w", "b", "m"], "y", **attrs)
        out = "y"
        if post == "lut":
            b.const("t", rng.integers(-127, 128, 256).astype(np.int8))
            b.node("QLut", ["y", "t"], "z")
            out = "z"
        b.output(out)
        feeds = {"x": (rng.standard_normal((n, c, hw, hw)) * 2).astype(np.float32)}
        return b.graph(), feeds, out

    g, feeds, out = graph()
    cmod, got, want = device_run(g, feeds, ctx=hip_ctx)
    assert [l.kind for l in cmod.module.plan] == ["qconv_first"]
    if cap:
        assert cmod.module.plan[0].grid[0] == cap
    np.testing.assert_array_equal(got[out], want[out])
    g2, _, _ = graph()
    _, got2, want2 = device_run(g2, feeds, ctx=hip_ctx, fuse_int8_epilogues=False)
    np.testing.assert_array_equal(got[out], got2[out])
    v = want2["y"].astype(int) if "y" in want2 else want[out].astype(int)
    assert v.std() > 3 and np.mean(np.abs(v) == 127) < 0.5
