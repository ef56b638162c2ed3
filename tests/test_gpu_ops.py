"""Device parity of the ops the reference ran on the host (its host-fallback
list, mdlc/codegen/cuda/emit.py:32-35 and :175-180): grouped convolution
with more than one channel per group, and average pooling in both
count_include_pad modes. Each runs as one device launch and is held to the
oracle (mdlc/runtime/ops.py:56-81, :128-146) at rtol 1e-4 / atol 1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest

from gpu_util import assert_close, device_run
from mdlc_amd.tools.graph_builder import GraphBuilder

pytestmark = pytest.mark.gpu


def _grouped_graph(n, c, h, w, oc, kh, kw, stride, pads, dil, group, *, bias=True, act="Relu",
                   residual=False, seed=4):
    rng = np.random.default_rng(seed)
    b = GraphBuilder("gconv")
    b.input("x", (n, c, h, w))
    icg = c // group
    b.const("w", (rng.standard_normal((oc, icg, kh, kw)) * np.sqrt(2.0 / (icg * kh * kw)))
            .astype(np.float32))
    ins = ["x", "w"]
    if bias:
        b.const("b", (rng.standard_normal(oc) * 0.1).astype(np.float32))
        ins.append("b")
    out = "y" if act is None and not residual else "pre"
    b.node("Conv", ins, out, kernel_shape=[kh, kw], strides=list(stride), pads=list(pads),
           dilations=list(dil), group=group)
    feeds = {"x": rng.standard_normal((n, c, h, w)).astype(np.float32)}
    if residual:
        oh = (h + pads[0] + pads[2] - dil[0] * (kh - 1) - 1) // stride[0] + 1
        ow = (w + pads[1] + pads[3] - dil[1] * (kw - 1) - 1) // stride[1] + 1
        b.input("r", (n, oc, oh, ow))
        b.node("Add", [out, "r"], "sum")
        b.node("Relu", ["sum"], "y")
        feeds["r"] = rng.standard_normal((n, oc, oh, ow)).astype(np.float32)
    elif act is not None:
        b.node(act, [out], "y")
    b.output("y")
    return b.graph(), feeds


GROUPED = [
    # n, c, h, w, oc, kh, kw, stride, pads(t,l,b,r), dil, group
    (1, 4, 9, 9, 8, 3, 3, (2, 2), (0, 0, 0, 0), (1, 1), 2),       # the oracle's own grouped case
    (2, 6, 10, 7, 9, 3, 2, (2, 1), (1, 0, 2, 1), (1, 2), 3),       # asymmetric pads, dilation
    (3, 8, 12, 12, 8, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 4),      # 2 channels per group
    (2, 64, 14, 14, 64, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 2),    # 32 channels/group: tap-major K
    (4, 128, 8, 8, 128, 3, 3, (2, 2), (1, 1, 1, 1), (1, 1), 32),   # ResNeXt-style cardinality 32
    (2, 16, 9, 9, 24, 1, 1, (1, 1), (0, 0, 0, 0), (1, 1), 4),      # grouped 1x1
]


@pytest.mark.parametrize("mode", ["implicit", "im2col"])
@pytest.mark.parametrize("case", GROUPED, ids=lambda c: "g{}_c{}_oc{}_k{}x{}".format(c[10], c[1], c[4], c[5], c[6]))
def test_grouped_conv_matches_oracle(case, mode, hip_ctx):
    g, feeds = _grouped_graph(*case)
    c, got, want = device_run(g, feeds, conv_mode=mode, ctx=hip_ctx)
    kinds = [l.kind for l in c.module.plan]
    assert kinds == ["gconv"], kinds
    assert c.module.plan[0].grid[1] == case[10]
    assert_close("y", got["y"], want["y"])


@pytest.mark.parametrize("bias,act", [(False, None), (True, "Sigmoid")])
def test_grouped_conv_epilogues(bias, act, hip_ctx):
    g, feeds = _grouped_graph(2, 12, 11, 11, 18, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 3,
                              bias=bias, act=act, seed=6)
    _, got, want = device_run(g, feeds, ctx=hip_ctx)
    assert_close("y", got["y"], want["y"])


@pytest.mark.parametrize("fold", [True, False])
def test_grouped_conv_residual_fold(fold, hip_ctx):
    """A residual Add + Relu after a grouped conv folds into its epilogue
    (each group reads its own channels of the residual) or runs as its own
    elementwise group; both match the oracle."""
    g, feeds = _grouped_graph(2, 16, 10, 10, 16, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 4,
                              act=None, residual=True, seed=8)
    c, got, want = device_run(g, feeds, ctx=hip_ctx, fuse_residual=fold)
    assert ("elementwise" in [l.kind for l in c.module.plan]) != fold
    assert_close("y", got["y"], want["y"])


POOLS = [
    # kernel, strides, pads (t, l, b, r), ceil
    ((3, 3), (2, 2), (1, 1, 1, 1), 0),
    ((2, 2), (2, 2), (0, 0, 0, 0), 0),
    ((3, 2), (1, 3), (1, 0, 2, 1), 0),
    ((5, 5), (1, 1), (2, 2, 2, 2), 0),
    ((3, 3), (2, 2), (0, 0, 0, 0), 1),          # ceil mode where it divides evenly (oracle limit)
    ((7, 7), (1, 1), (0, 0, 0, 0), 0),          # whole 7x7 plane
]


@pytest.mark.parametrize("cip", [0, 1])
@pytest.mark.parametrize("pool", POOLS, ids=lambda p: "k{}x{}_s{}x{}_p{}{}{}{}_c{}".format(
    *p[0], *p[1], *p[2], p[3]))
def test_average_pool_matches_oracle(pool, cip, hip_ctx):
    (kh, kw), (sh, sw), pads, ceil = pool
    rng = np.random.default_rng(13)
    b = GraphBuilder("ap")
    shape = (2, 5, 7, 7) if (kh, kw) == (7, 7) else (3, 5, 15, 13)
    b.input("x", shape)
    b.node("AveragePool", ["x"], "y", kernel_shape=[kh, kw], strides=[sh, sw], pads=list(pads),
           count_include_pad=cip, ceil_mode=ceil)
    b.output("y")
    feeds = {"x": rng.standard_normal(shape).astype(np.float32)}
    c, got, want = device_run(b.graph(), feeds, ctx=hip_ctx)
    assert [l.kind for l in c.module.plan] == ["avgpool"]
    assert_close("y", got["y"], want["y"])


# ----- Softmax, Transpose, Pad, Concat ------------------------------------------------

def _one_op(shape, op, attrs=None, extra_consts=(), seed=17, nin=1, shapes=None):
    rng = np.random.default_rng(seed)
    b = GraphBuilder(op.lower())
    feeds, ins = {}, []
    for i, shp in enumerate(shapes or [shape] * nin):
        name = f"x{i}"
        b.input(name, shp)
        feeds[name] = (rng.standard_normal(shp) * 3).astype(np.float32)
        ins.append(name)
    for name, arr in extra_consts:
        b.const(name, arr)
        ins.append(name)
    b.node(op, ins, "y", **(attrs or {}))
    b.output("y")
    return b.graph(), feeds


@pytest.mark.parametrize("shape,axis", [((4, 1000), -1), ((4, 1000), 1), ((2, 3, 5, 7), 1),
                                        ((2, 3, 5, 7), 3), ((2, 3, 5, 7), 0), ((3, 4097), -1),
                                        ((6, 1), -1)])
def test_softmax_matches_oracle(shape, axis, hip_ctx):
    g, feeds = _one_op(shape, "Softmax", {"axis": axis})
    c, got, want = device_run(g, feeds, ctx=hip_ctx)
    assert [l.kind for l in c.module.plan] == ["softmax"]
    assert_close("y", got["y"], want["y"])
    np.testing.assert_allclose(got["y"].sum(axis=axis), 1.0, rtol=1e-5)


@pytest.mark.parametrize("shape,perm", [((2, 3, 4, 5), (0, 2, 3, 1)), ((2, 3, 4, 5), (3, 1, 0, 2)),
                                        ((2, 3, 4, 5), None), ((2, 3, 1, 4, 2, 3), (5, 0, 4, 1, 3, 2)),
                                        ((7, 9), (1, 0))])
def test_transpose_is_exact(shape, perm, hip_ctx):
    g, feeds = _one_op(shape, "Transpose", {"perm": list(perm)} if perm else {})
    c, got, want = device_run(g, feeds, ctx=hip_ctx)
    assert [l.kind for l in c.module.plan] == ["transpose"]
    np.testing.assert_array_equal(got["y"], want["y"])


@pytest.mark.parametrize("mode,value", [("constant", 0.0), ("constant", -1.5), ("edge", 0.0),
                                        ("reflect", 0.0)])
@pytest.mark.parametrize("as_input", [True, False])
def test_pad_is_exact(mode, value, as_input, hip_ctx):
    shape = (2, 3, 6, 5)
    pads = [0, 1, 2, 0, 0, 0, 3, 4]
    if as_input:
        g, feeds = _one_op(shape, "Pad", {"mode": mode},
                           extra_consts=[("pads", np.array(pads, np.int64)),
                                         ("value", np.array(value, np.float32))])
    else:
        g, feeds = _one_op(shape, "Pad", {"mode": mode, "pads": pads, "value": value})
    c, got, want = device_run(g, feeds, ctx=hip_ctx)
    assert [l.kind for l in c.module.plan] == ["pad"]
    assert got["y"].shape == (2, 4, 11, 9)
    np.testing.assert_array_equal(got["y"], want["y"])


@pytest.mark.parametrize("shapes,axis", [([(2, 3, 4, 5), (2, 1, 4, 5), (2, 6, 4, 5)], 1),
                                         ([(1, 3, 4, 5), (3, 3, 4, 5)], 0),
                                         ([(2, 3, 4, 5), (2, 3, 4, 2)], -1),
                                         ([(8, 1000), (8, 24)], 1)])
def test_concat_is_exact(shapes, axis, hip_ctx):
    g, feeds = _one_op(None, "Concat", {"axis": axis}, shapes=shapes)
    c, got, want = device_run(g, feeds, ctx=hip_ctx)
    assert [l.kind for l in c.module.plan] == ["concat"] * len(shapes)
    np.testing.assert_array_equal(got["y"], want["y"])
