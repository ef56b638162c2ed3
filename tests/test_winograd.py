"""Host side of the Winograd F(2x2, 3x3) convolution, on the CPU.

The filter transform the emitter packs is pinned by the algorithm's own
identity: with the textbook input and output transforms (Lavin & Gray,
"Fast Algorithms for Convolutional Neural Networks", 2016, F(2x2, 3x3)),
A^T [U (.) (B^T d B)] A summed over channels must equal the direct
correlation of the reference's Conv (mdlc/runtime/ops.py:56-81), to float64
rounding, for every 4x4 window. A wrong G row, a swapped (a, b) position
order or a transposed filter fails it. The emitter's choices (which convs,
how many channel slices, padded layouts) are checked on the plan.
"""

from __future__ import annotations

import numpy as np
import pytest

from mdlc_amd.codegen.hip.emit import wino_filter_transform
from mdlc_amd.codegen.schedule import wino_pays, wino_slices
from mdlc_amd.compiler import compile_graph
from mdlc_amd.tools.graph_builder import GraphBuilder

BT = np.array([[1, 0, -1, 0], [0, 1, 1, 0], [0, -1, 1, 0], [0, 1, 0, -1]], np.float64)
AT = np.array([[1, 1, 1, 0], [0, 1, -1, -1]], np.float64)


def _direct(x, w):
    """Valid 3x3 correlation, float64: y[o, i, j] = sum_c,u,v w[o,c,u,v] x[c,i+u,j+v]."""
    C, H, W = x.shape
    y = np.zeros((w.shape[0], H - 2, W - 2))
    for u in range(3):
        for v in range(3):
            y += np.einsum("oc,chw->ohw", w[:, :, u, v], x[:, u:u + H - 2, v:v + W - 2])
    return y


@pytest.mark.parametrize("oc,c", [(1, 1), (3, 5), (8, 16)])
def test_filter_transform_reproduces_direct_conv(oc, c):
    rng = np.random.default_rng(oc * 10 + c)
    w = rng.standard_normal((oc, c, 3, 3))
    x = rng.standard_normal((c, 8, 6))
    u = wino_filter_transform(w.astype(np.float32)).astype(np.float64).reshape(4, 4, oc, c)
    # recompute U in float64 so the identity is checked to float64 rounding;
    # the packed float32 U must be that, rounded once
    w32 = w.astype(np.float32).astype(np.float64)
    G = np.array([[1, 0, 0], [0.5, 0.5, 0.5], [0.5, -0.5, 0.5], [0, 0, 1]])
    u64 = np.einsum("ai,ocij,bj->aboc", G, w32, G)
    assert np.array_equal(u, u64.astype(np.float32).astype(np.float64))
    want = _direct(x, w32)
    got = np.zeros_like(want)
    for ty in range(3):
        for tx in range(2):
            d = x[:, 2 * ty:2 * ty + 4, 2 * tx:2 * tx + 4]                  # [c][4][4]
            v = np.einsum("ai,cij,bj->abc", BT, d, BT)                       # B^T d B
            m = np.einsum("aboc,abc->abo", u64, v)                           # sum over c
            got[:, 2 * ty:2 * ty + 2, 2 * tx:2 * tx + 2] = np.einsum("ia,abo,jb->oij", AT, m, AT)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12 * max(1.0, np.abs(want).max()))


def test_slices_fill_the_chip_without_starving_slices():
    # ResNet-18 at batch 32: rounds of workgroups x chunks per slice is
    # 2 x 8, 1 x 16, 1 x 16, 1 x 16 chunk times; more slices would not
    # lower it (stage 2: 2 slices = 2 rounds x 8)
    assert [wino_slices(oc, t, oc) for oc, t in
            [(64, 25088), (128, 6272), (256, 1568), (512, 512)]] == [1, 1, 2, 4]
    assert wino_slices(512, 16, 512) == 16                  # batch 1: 4 chunks per slice
    assert wino_slices(64, 10, 24) == 1                      # too few chunks to split


def test_auto_choice_takes_winograd_only_for_grids_that_fill_the_chip():
    # ResNet-18's 3x3 stride-1 layers: every stage at batch 32, none at batch 1
    layers = [(64, 784, 64), (128, 196, 128), (256, 49, 256), (512, 16, 512)]
    assert all(wino_pays(oc, 32 * t, c) for oc, t, c in layers)
    assert not any(wino_pays(oc, t, c) for oc, t, c in layers)
    from mdlc_amd.tools.build_resnet18 import build_resnet18, make_input
    for batch, n in ((32, 13), (1, 0)):
        c = compile_graph(build_resnet18(batch=batch), feeds={"input": make_input(batch)})
        assert sum(l.kind == "wino" for l in c.module.plan) == n
    with pytest.raises(ValueError, match="winograd"):
        compile_graph(build_resnet18(batch=1), winograd="yes")


def _graph(c, oc, h, w, k=3, s=1, d=1, group=1):
    rng = np.random.default_rng(0)
    b = GraphBuilder("g")
    b.input("x", (1, c, h, w))
    b.const("w", rng.standard_normal((oc, c // group, k, k)).astype(np.float32))
    p = d * (k // 2)
    b.node("Conv", ["x", "w"], "y", kernel_shape=[k, k], strides=[s, s], dilations=[d, d],
           pads=[p] * 4, group=group)
    b.output("y")
    return b.graph(), {"x": rng.standard_normal((1, c, h, w)).astype(np.float32)}


@pytest.mark.parametrize("k,s,d,group,wino", [(3, 1, 1, 1, True), (3, 2, 1, 1, False),
                                             (3, 1, 2, 1, False), (5, 1, 1, 1, False),
                                             (3, 1, 1, 2, False)])
def test_only_plain_3x3_stride1_convs_take_winograd(k, s, d, group, wino):
    g, feeds = _graph(16, 16, 9, 9, k, s, d, group)
    kinds = [l.kind for l in compile_graph(g, feeds=feeds, winograd=True).module.plan]
    assert ("wino" in kinds) == wino, kinds
    g, feeds = _graph(16, 16, 9, 9, k, s, d, group)
    assert "wino" not in [l.kind for l in compile_graph(g, feeds=feeds, winograd=False).module.plan]


def test_packed_filters_are_padded_to_whole_blocks_and_slices():
    g, feeds = _graph(200, 130, 6, 10)
    c = compile_graph(g, feeds=feeds, winograd=True)
    (l,) = [l for l in c.module.plan if l.kind == "wino"]
    m = l.meta
    # 25 chunks over 8 slices: 4 a slice, 7 slices (no empty one), 28 chunks packed
    assert (m["OCP"], m["nchunk"], l.grid[1], m["CP"]) == (192, 4, 7, 224)
    img = c.module.device_constants[l.inputs[0]]
    assert img.shape == (3, 28, 2, 4, 2, 64, 2, 4)     # [ocb][chunk][h][blk][j][lane][slot][4]
    # undo the per-lane slot swizzle (slot s holds quartet s ^ sw), then back to [16][OCP][CP]
    lanes = np.arange(64)
    sw = ((lanes >> 2) ^ (lanes >> 3)) & 1
    img = img[:, :, :, :, :, lanes[:, None], np.arange(2)[None, :] ^ sw[:, None]]
    # axes: ocb, chunk, h, blk, j, lk, li, q, e -> xi = 8h + 4q + e, oc = (ocb, blk, li), k = (chunk, j, lk)
    u = img.reshape(3, 28, 2, 4, 2, 4, 16, 2, 4).transpose(2, 7, 8, 0, 3, 6, 1, 4, 5).reshape(16, 192, 224)
    assert not u[:, 130:, :].any() and not u[:, :, 200:].any()
    w = wino_filter_transform(c.graph.initializers["w"])
    np.testing.assert_array_equal(u[:, :130, :200], w)
    # the A operand lane 37 (lk 2, li 5) of a half-1 wave reads for blk 2, j = 1 in
    # quartet q = 1: positions 12-15 of oc 32 + 5 = 37, channel 8 * 3 + 2 + 4 = 30 of chunk 3
    raw = c.module.device_constants[l.inputs[0]]
    q, lane = 1, 37
    slot = q ^ (((lane >> 2) ^ (lane >> 3)) & 1)
    np.testing.assert_array_equal(raw[0, 3, 1, 2, 1, lane, slot], w[12:16, 37, 30])
    (r,) = [r for r in c.module.plan if r.kind == "splitk_reduce"]
    assert r.meta["S"] == 7 and c.module.scratch_shapes[r.inputs[0]] == (7 * 130, 60)
