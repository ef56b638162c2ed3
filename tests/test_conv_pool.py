"""The fused small-channel conv + 3x3 stride-2 max pool, host side, on the
CPU: when the fold fires, that the folded graph means the same thing, and
the kernel's index arithmetic replayed in NumPy — its patch (every input
row of the band, every column), the per-lane k offsets, the 16x16x4 MFMA
lane layout, the vertical maxima in registers, the horizontal maxima across
lanes (DPP row shifts) with the previous block's last column rotated in,
and the pooled
stores — against conv -> activation -> pool, so a wrong offset, lane or
carry fails here before any device run."""

from __future__ import annotations

import numpy as np
import pytest

import mdlc_amd.codegen.schedule as S
from mdlc_amd.codegen.schedule import conv_pool_band
from mdlc_amd.compiler import compile_graph
from mdlc_amd.tools.build_resnet18 import build_resnet18
from mdlc_amd.tools.graph_builder import GraphBuilder
from oracle import ops
from oracle.reference import run_reference


def _graph(n, c, h, w, oc, k, s, p, act="Relu", bias=True, seed=0):
    rng = np.random.default_rng(seed)
    b = GraphBuilder("convpool")
    b.input("x", (n, c, h, w))
    b.const("w", rng.standard_normal((oc, c, k, k)).astype(np.float32))
    ins = ["x", "w"]
    if bias:
        b.const("b", rng.standard_normal(oc).astype(np.float32))
        ins.append("b")
    b.node("Conv", ins, "y", kernel_shape=[k, k], strides=[s, s], pads=[p] * 4)
    last = "y"
    if act:
        b.node(act, ["y"], "a", **({"min": 0.0, "max": 6.0} if act == "Clip" else {}))
        last = "a"
    b.node("MaxPool", [last], "z", kernel_shape=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1])
    b.output("z")
    return b.graph(), {"x": rng.standard_normal((n, c, h, w)).astype(np.float32)}


def _replay(x, packed, bias, geo, R, act):
    """The kernel's arithmetic for every workgroup and wave in float64, the
    MFMA as D[i][j] += sum_k A[i][k] B[k][j] with lane l = 16 lk + li giving
    A[li][lk] and B[lk][li] and holding D[4 lk + r][li] in register r."""
    N, C, H, W, OC, KH, KW, SH, SW, PT, PL = geo
    OH, OW = (H + 2 * PT - KH) // SH + 1, (W + 2 * PL - KW) // SW + 1
    NBX, PH, PW = OW // 16, OH // 2, OW // 2
    NR, K = 2 * R + 1, C * KH * KW
    PR, PC = (NR - 1) * SH + KH, (OW - 1) * SW + KW
    NS = -(-K // 4)
    bands = PH // R
    lanes = np.arange(64)
    li, lk = lanes & 15, lanes >> 4
    k = 4 * np.arange(NS)[:, None] + lk[None, :]
    k = np.where(k < K, k, 0)
    c, t = k // (KH * KW), k % (KH * KW)
    koff = (c * PR + t // KW) * PC + t % KW                    # [step][lane]
    ror1 = (lanes & 48) | ((li + 15) & 15)                  # lane i <- (i - 1) mod 16
    shr1 = (lanes & 48) | np.maximum(li - 1, 0)             # lane i <- i - 1
    shl1 = (lanes & 48) | np.minimum(li + 1, 15)            # lane i <- i + 1
    y = np.full((N, OC, PH, PW), np.nan)
    for wg in range(N * bands):
        n, kb = divmod(wg, bands)
        ih0 = (2 * R * kb - 1) * SH - PT
        row = np.arange(C * PR)
        cc, ih = row // PR, ih0 + row % PR
        iw = np.arange(PC) - PL
        ok = ((ih >= 0) & (ih < H))[:, None] & ((iw >= 0) & (iw < W))[None, :]
        patch = np.where(ok, x[n, cc[:, None], np.clip(ih, 0, H - 1)[:, None],
                               np.clip(iw, 0, W - 1)[None, :]], 0.0).reshape(-1)
        for blk in range(packed.shape[0]):
            wr = packed[blk]                                   # [step][lane]
            vprev = np.full((R, 64, 4), -np.inf)
            for bx in range(NBX):
                base = (16 * bx + li) * SW
                acc = np.zeros((NR, 64, 4))
                for s in range(NS):
                    A = np.zeros((16, 4))
                    A[li, lk] = wr[s]
                    for i in range(NR):
                        idx = koff[s] + base + i * SH * PC
                        assert idx.min() >= 0 and idx.max() < patch.size
                        B = np.zeros((4, 16))
                        B[lk, li] = patch[idx]
                        D = A @ B
                        for r in range(4):
                            acc[i, :, r] += D[4 * lk + r, li]
                for j in range(R):
                    v = np.maximum(acc[2 * j + 1], acc[2 * j + 2])
                    if kb > 0 or j > 0:
                        v = np.maximum(acc[2 * j], v)
                    # row_ror:1 of the previous block into lane 0, row_shr:1 /
                    # row_shl:1 within each row of 16 (a lane without a source
                    # keeps the old operand)
                    carry = vprev[j][ror1]
                    left = np.where((li == 0)[:, None], carry, v[shr1])
                    right = np.where((li == 15)[:, None], v, v[shl1])
                    m = np.maximum(np.maximum(left, v), right)
                    vprev[j] = v
                    for ln in range(0, 64, 2):
                        for r in range(4):
                            _store(y, bias, act, OC, n, blk * 16 + 4 * lk[ln] + r, R * kb + j,
                                   8 * bx + li[ln] // 2, m[ln, r])
    return y


def _store(y, bias, act, OC, n, oc, py, px, m):
    if oc < OC:
        val = m + (bias[oc] if bias is not None else 0.0)
        if act == "Relu":
            val = max(val, 0.0)
        elif act == "Clip":
            val = min(max(val, 0.0), 6.0)
        y[n, oc, py, px] = val


@pytest.fixture
def few_cus(monkeypatch):
    """Let small test shapes take the fused kernel (it needs a band per CU)."""
    monkeypatch.setattr(S, "CUS", 2)


@pytest.mark.parametrize("case", [(2, 3, 32, 32, 20, 7, 2, 3, "Relu", True),
                                  (1, 3, 64, 64, 64, 7, 2, 3, "Relu", True),
                                  (1, 3, 96, 96, 16, 7, 2, 3, "Relu", True),
                                  (1, 2, 32, 32, 16, 3, 1, 1, "Clip", False),
                                  (1, 1, 64, 32, 40, 5, 2, 2, None, True)],
                         ids=lambda c: "x".join(map(str, c)))
def test_index_replay_matches_conv_act_pool(case, few_cus):
    n, c, h, w, oc, k, s, p, act, bias = case
    g, feeds = _graph(n, c, h, w, oc, k, s, p, act=act, bias=bias)
    comp = compile_graph(g, feeds=feeds)
    (launch,) = comp.module.plan
    assert launch.kind == "conv_pool"
    R = launch.meta["band"]
    packed = comp.module.device_constants[launch.inputs[1]].astype(np.float64)
    b = g.initializers["b"].astype(np.float64) if bias else None
    x64 = feeds["x"].astype(np.float64)
    got = _replay(x64, packed, b, (n, c, h, w, oc, k, k, s, s, p, p), R, act)
    conv = ops.conv(x64, g.initializers["w"].astype(np.float64), b, strides=[s, s], pads=[p] * 4,
                    dilations=[1, 1], group=1)
    if act == "Relu":
        conv = np.maximum(conv, 0.0)
    elif act == "Clip":
        conv = np.clip(conv, 0.0, 6.0)
    want = ops.maxpool(conv, kernel=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1])
    assert not np.isnan(got).any()
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)


def test_folded_graph_means_the_same(few_cus):
    g, feeds = _graph(2, 3, 32, 32, 24, 7, 2, 3)
    want = run_reference(g, feeds)["z"]
    comp = compile_graph(g, feeds=feeds)
    (node,) = comp.graph.nodes
    assert node.attrs["maxpool"]["strides"] == [2, 2] and node.outputs == ["z"]
    np.testing.assert_array_equal(run_reference(comp.graph, feeds)["z"], want)


def test_where_the_fold_fires():
    assert conv_pool_band(3, 7, 7, 2, 2, 1, 1, 32, 112, 112) == 7      # ResNet-18 stem, b=32
    assert conv_pool_band(3, 7, 7, 2, 2, 1, 1, 16, 112, 112) is None   # 128 bands < 256 CUs
    assert conv_pool_band(5, 7, 7, 2, 2, 1, 1, 64, 112, 112) is None   # too many channels
    assert conv_pool_band(3, 7, 7, 2, 2, 1, 1, 64, 112, 104) is None   # OW % 16
    assert conv_pool_band(3, 3, 3, 2, 2, 2, 2, 64, 112, 112) is None   # dilated
    kinds = [l.kind for l in compile_graph(build_resnet18(batch=32)).module.plan]
    assert kinds[0] == "conv_pool" and "maxpool" not in kinds
    kinds = [l.kind for l in compile_graph(build_resnet18(batch=1)).module.plan]
    assert kinds[:2] == ["conv_smallc", "maxpool"]
    kinds = [l.kind for l in compile_graph(build_resnet18(batch=32), fuse_pool=False).module.plan]
    assert kinds[:2] == ["conv_smallc", "maxpool"]


def test_fold_refuses_other_consumers_and_windows(few_cus):
    g, feeds = _graph(2, 3, 32, 32, 24, 7, 2, 3, act="Sigmoid")      # not non-decreasing in float
    assert [l.kind for l in compile_graph(g, feeds=feeds).module.plan][-1] == "maxpool"
    b = GraphBuilder("twice")
    b.input("x", (2, 3, 32, 32))
    b.const("w", np.ones((16, 3, 7, 7), np.float32))
    b.node("Conv", ["x", "w"], "y", kernel_shape=[7, 7], strides=[2, 2], pads=[3] * 4)
    b.node("MaxPool", ["y"], "z", kernel_shape=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1])
    b.output("z")
    b.output("y")                                                    # the conv output is needed
    g = b.graph()
    assert "conv_pool" not in [l.kind for l in compile_graph(g).module.plan]
