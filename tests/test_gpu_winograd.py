"""Device parity of the Winograd F(2x2, 3x3) convolution (compile option
``winograd``): 3x3 stride-1 convs of the reference's Conv op
(mdlc/runtime/ops.py:56-81) at odd and even sizes, channel counts off the
kernel's 8-channel chunks and 64-channel blocks, asymmetric padding, every
epilogue (bias, activation, folded residual) and the channel-split form with
its ordered reduce, each held to the oracle at rtol 1e-4 / atol 1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest

from gpu_util import assert_close, device_run
from mdlc_amd.tools.graph_builder import GraphBuilder

pytestmark = pytest.mark.gpu


def _conv_graph(n, c, h, w, oc, pads, *, bias=True, act="Relu", residual=False, seed=7):
    rng = np.random.default_rng(seed)
    b = GraphBuilder("wino")
    b.input("x", (n, c, h, w))
    b.const("w", (rng.standard_normal((oc, c, 3, 3)) * np.sqrt(2.0 / (9 * c))).astype(np.float32))
    ins = ["x", "w"]
    if bias:
        b.const("b", (rng.standard_normal(oc) * 0.1).astype(np.float32))
        ins.append("b")
    out = "y" if act is None and not residual else "pre"
    b.node("Conv", ins, out, kernel_shape=[3, 3], strides=[1, 1], pads=list(pads))
    feeds = {"x": rng.standard_normal((n, c, h, w)).astype(np.float32)}
    if residual:
        oh, ow = h + pads[0] + pads[2] - 2, w + pads[1] + pads[3] - 2
        b.input("r", (n, oc, oh, ow))
        b.node("Add", [out, "r"], "sum")
        b.node("Relu", ["sum"], "y")
        feeds["r"] = rng.standard_normal((n, oc, oh, ow)).astype(np.float32)
    elif act is not None:
        b.node(act, [out], "y")
    b.output("y")
    return b.graph(), feeds


CASES = [
    # n, c, h, w, oc, pads (t, l, b, r), channel slices the grid gets
    (2, 64, 56, 56, 64, (1, 1, 1, 1), 2),     # ResNet-18 stage 1 at batch 2
    (3, 20, 13, 11, 40, (1, 1, 1, 1), 1),     # odd sizes, partial chunk and channel block
    (1, 12, 9, 15, 100, (0, 1, 2, 0), 1),     # asymmetric pads, two channel blocks
    (1, 36, 5, 5, 64, (0, 0, 0, 0), 1),       # valid conv, 3x3 output (odd tile edge)
    (1, 5, 8, 8, 7, (1, 1, 1, 1), 1),         # one partial chunk
    (2, 256, 7, 7, 72, (1, 1, 1, 1), 8),      # small grid: channel sum over 8 slices
    (1, 200, 6, 10, 130, (2, 1, 0, 2), 7),    # slices with a partial last chunk
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "n{}_c{}_{}x{}_oc{}_p{}".format(
    c[0], c[1], c[2], c[3], c[4], "".join(map(str, c[5]))))
def test_winograd_conv_matches_oracle(case, hip_ctx):
    *shape, pads, slices = case
    g, feeds = _conv_graph(*shape, pads)
    c, got, want = device_run(g, feeds, ctx=hip_ctx, winograd=True)
    wino = [l for l in c.module.plan if l.kind == "wino"]
    assert len(wino) == 1 and wino[0].grid[1] == slices, [(l.kind, l.grid) for l in c.module.plan]
    assert_close("y", got["y"], want["y"])


@pytest.mark.parametrize("bias,act", [(False, None), (True, "Sigmoid"), (False, "LeakyRelu")])
@pytest.mark.parametrize("split", [False, True])
def test_winograd_epilogues(bias, act, split, hip_ctx):
    shape = (2, 256, 7, 7, 64) if split else (2, 24, 17, 17, 48)
    g, feeds = _conv_graph(*shape, (1, 1, 1, 1), bias=bias, act=act, seed=11)
    c, got, want = device_run(g, feeds, ctx=hip_ctx, winograd=True)
    assert (c.module.plan[0].grid[1] > 1) == split
    assert_close("y", got["y"], want["y"])


@pytest.mark.parametrize("split", [False, True])
def test_winograd_residual_fold(split, hip_ctx):
    """Add + Relu after the conv folds into the Winograd epilogue, or into the
    reduce of the split form: one or two launches, same values."""
    shape = (2, 256, 7, 7, 64) if split else (2, 32, 14, 14, 32)
    g, feeds = _conv_graph(*shape, (1, 1, 1, 1), residual=True, seed=12)
    c, got, want = device_run(g, feeds, ctx=hip_ctx, winograd=True)
    assert [l.kind for l in c.module.plan] == (["wino", "splitk_reduce"] if split else ["wino"])
    assert_close("y", got["y"], want["y"])


def test_winograd_skips_other_convs(hip_ctx):
    """Strided, dilated and non-3x3 convs keep the implicit GEMM."""
    rng = np.random.default_rng(3)
    b = GraphBuilder("mixed")
    b.input("x", (1, 16, 12, 12))
    for i, (k, s, d) in enumerate([(3, 2, 1), (3, 1, 2), (1, 1, 1)]):
        b.const(f"w{i}", (rng.standard_normal((16, 16, k, k)) * 0.2).astype(np.float32))
        p = d * (k // 2)
        b.node("Conv", ["x" if i == 0 else f"y{i - 1}", f"w{i}"], f"y{i}", kernel_shape=[k, k],
               strides=[s, s], dilations=[d, d], pads=[p] * 4)
    b.output("y2")
    feeds = {"x": rng.standard_normal((1, 16, 12, 12)).astype(np.float32)}
    c, got, want = device_run(b.graph(), feeds, ctx=hip_ctx, winograd=True)
    assert "wino" not in {l.kind for l in c.module.plan}
    assert_close("y2", got["y2"], want["y2"])
