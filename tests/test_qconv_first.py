"""The first int8 conv with its input quantization folded in, host side, on
the CPU: the kernel's arithmetic replayed in NumPy — the band's quantized
patch (one word of channel codes per input pixel, zeros at the padding), the
per-lane tap offsets, the packed weight fragments, the 16x16x64 int8 MFMA
lane layout, the requant / lookup epilogue and the band's contiguous
channels-last store — against the oracle's QuantizeLinear -> QConv (-> QLut)
graph, bit for bit, so a wrong offset, lane, byte or band fails here before
any device run."""

from __future__ import annotations

import numpy as np
import pytest

import mdlc_amd.codegen.schedule as S
from mdlc_amd.codegen.schedule import qconv_first_band
from mdlc_amd.compiler import compile_graph
from mdlc_amd.tools.graph_builder import GraphBuilder
from oracle.reference import run_reference


def _graph(n, c, hw, oc, k, s, post, seed=21):
    rng = np.random.default_rng(seed)
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
    x = (rng.standard_normal((n, c, hw, hw)) * 2).astype(np.float32)
    x.flat[::97] = 6.0                                       # some codes clamp at 127
    return b.graph(), {"x": x}, out


def _f32(v):
    return np.asarray(v, np.float32)


def _replay(x, inv_s, wdev, bias, mult, table, geo, R, lo):
    """Every band and wave of the kernel in NumPy (which workgroup takes a
    band does not change its arithmetic). The MFMA is
    D[i][j] = sum over lane groups g and the 16 bytes of lane (i, g) of the
    row operand times the same bytes of lane (j, g) of the column operand,
    lane l = 16 g + i; D[4 g + r][i] is register r of lane 16 g + i."""
    N, C, H, W, OC, KH, KW, SH, SW, PT, PL = geo
    OH, OW = (H + 2 * PT - KH) // SH + 1, (W + 2 * PL - KW) // SW + 1
    T, NOB, NS = KH * KW, -(-OC // 16), -(-(KH * KW) // 16)
    PR, PCW = (R - 1) * SH + KH, (OW - 1) * SW + KW
    NP, BANDS = R * OW, -(-OH // R)
    lanes = np.arange(64)
    li, lk = lanes & 15, lanes >> 4
    wf = wdev.reshape(NOB, NS, 64, 4)                            # int32 words
    t = 16 * np.arange(NS)[:, None, None] + 4 * lk[None, :, None] + np.arange(4)[None, None, :]
    toff = np.where(t < T, (t // KW) * PCW + t % KW, 0)          # [step][lane][j]
    y = np.zeros((N, OH, OW, OC), np.int8)
    written = np.zeros(y.shape, bool)
    for bi in range(N * BANDS):
        n, band = divmod(bi, BANDS)
        oh0 = band * R
        e = np.arange(PR * PCW)
        ih, iw = oh0 * SH - PT + e // PCW, e % PCW - PL
        ok = (ih >= 0) & (ih < H) & (iw >= 0) & (iw < W)
        codes = np.zeros((PR * PCW, 4), np.int8)
        for c in range(C):
            v = np.where(ok, x[n, c, np.clip(ih, 0, H - 1), np.clip(iw, 0, W - 1)], np.float32(0))
            codes[:, c] = np.rint(np.clip(_f32(v * np.float32(inv_s)), -127, 127)).astype(np.int8)
        patch = codes.view(np.int32).reshape(-1)                 # byte c = channel c
        outs = np.zeros((NP, OC), np.int8)
        for g in range(-(-NP // 16)):
            p0 = 16 * g + li
            pv = p0 < NP
            p = np.where(pv, p0, 0)
            r, ow = p // OW, p % OW
            base = r * SH * PCW + ow * SW
            idx = base[None, :, None] + toff                     # [step][lane][j]
            assert idx.min() >= 0 and idx.max() < patch.size
            bfr = patch[idx].view(np.int8).reshape(NS, 64, 16).astype(np.int64)
            for ob in range(NOB):
                afr = wf[ob].view(np.int8).reshape(NS, 64, 16).astype(np.int64)
                D = np.zeros((16, 16), np.int64)
                for s in range(NS):
                    for grp in range(4):
                        D += afr[s, 16 * grp:16 * grp + 16] @ bfr[s, 16 * grp:16 * grp + 16].T
                for ln in range(64):
                    if not pv[ln] or 16 * ob + 4 * lk[ln] >= OC:
                        continue
                    for j in range(4):
                        oc = 16 * ob + 4 * lk[ln] + j
                        acc = np.int32(D[4 * lk[ln] + j, li[ln]] + bias[oc])
                        f = _f32(_f32(acc) * mult[oc])
                        code = int(np.rint(np.clip(f, lo, 127)))
                        outs[p[ln], oc] = table[code + 128] if table is not None else code
        rows = min(R, OH - oh0)
        y[n, oh0:oh0 + rows] = outs[:rows * OW].reshape(rows, OW, OC)
        written[n, oh0:oh0 + rows] = True
    assert written.all()
    return y


@pytest.fixture
def few_cus(monkeypatch):
    """Let the test shapes take bands of several rows (the band rule wants
    two workgroups a CU)."""
    monkeypatch.setattr(S, "CUS", 2)


@pytest.mark.parametrize("case", [(2, 3, 31, 24, 3, 2, "lut"), (1, 3, 16, 24, 3, 2, None),
                                  (2, 1, 9, 8, 5, 1, "lut"), (1, 4, 12, 16, 3, 1, "relu"),
                                  (3, 2, 7, 12, 3, 2, None), (1, 3, 20, 36, 3, 2, "lut")],
                         ids=lambda c: "n{}c{}hw{}oc{}k{}s{}_{}".format(*c))
def test_index_replay_matches_quantize_conv(case, few_cus):
    n, c, hw, oc, k, s, post = case
    g, feeds, out = _graph(n, c, hw, oc, k, s, post)
    want = run_reference(g, feeds)[out]
    comp = compile_graph(g, feeds=feeds)
    (launch,) = comp.module.plan
    assert launch.kind == "qconv_first"
    R = launch.meta["band"]
    consts = {**comp.graph.initializers, **comp.module.device_constants}
    wdev = consts[launch.inputs[1]]
    table = consts[launch.inputs[4]] if post == "lut" else None
    p = k // 2
    got = _replay(feeds["x"], launch.meta["inv_s"], wdev, consts[launch.inputs[2]],
                  consts[launch.inputs[3]], table, (n, c, hw, hw, oc, k, k, s, s, p, p), R,
                  0 if post == "relu" else -127)
    assert launch.grid == (min(n * -(-launch.meta["OH"] // R), 8 * S.CUS), 1, 1)
    np.testing.assert_array_equal(got.transpose(0, 3, 1, 2), want)


def test_band_rule():
    assert qconv_first_band(3, 3, 3, 2, 2, 32, 112, 112, 24) == 2     # RepViT stem, b=32: 1792 bands
    assert qconv_first_band(3, 3, 3, 2, 2, 1, 112, 112, 24) == 1      # b=1: one row a workgroup
    assert qconv_first_band(5, 3, 3, 2, 2, 32, 112, 112, 24) is None  # more than four channels
    assert qconv_first_band(3, 7, 7, 2, 2, 32, 112, 112, 24) is None  # 49 taps
    assert qconv_first_band(3, 3, 3, 2, 2, 32, 112, 112, 68) is None  # OC > 64
    assert qconv_first_band(3, 3, 3, 2, 2, 32, 112, 112, 18) is None  # OC % 4
    assert qconv_first_band(3, 3, 3, 1, 1, 1, 4096, 4096, 64) is None  # no band fits the LDS
