"""The direct small-channel convolution's host side, on the CPU: which convs
take it, the tile rule, and the packed weight layout. The kernel's index
arithmetic (patch offsets per pair, the 32x32x2 MFMA lane layout and the
epilogue's channel/pixel mapping) is replayed here in NumPy and compared with
a direct convolution, so a wrong offset or lane mapping fails on the CPU."""

from __future__ import annotations

import numpy as np
import pytest

from mdlc_amd.codegen.schedule import smallc_fits, smallc_pairs, smallc_tile
from mdlc_amd.compiler import compile_graph
from mdlc_amd.tools.graph_builder import GraphBuilder


def _graph(n, c, h, w, oc, k, s, p, seed=0):
    rng = np.random.default_rng(seed)
    b = GraphBuilder("smallc")
    b.input("x", (n, c, h, w))
    b.const("w", rng.standard_normal((oc, c, k, k)).astype(np.float32))
    b.node("Conv", ["x", "w"], "y", kernel_shape=[k, k], strides=[s, s], pads=[p] * 4)
    b.output("y")
    return b.graph(), {"x": rng.standard_normal((n, c, h, w)).astype(np.float32)}


def _direct(x, w, s, p):
    n, c, h, wd = x.shape
    oc, _, kh, kw = w.shape
    xp = np.pad(x, ((0, 0), (0, 0), (p, p), (p, p)))
    oh, ow = (h + 2 * p - kh) // s + 1, (wd + 2 * p - kw) // s + 1
    y = np.zeros((n, oc, oh, ow))
    for i in range(kh):
        for j in range(kw):
            win = xp[:, :, i:i + s * oh:s, j:j + s * ow:s]
            y += np.einsum("nchw,oc->nohw", win, w[:, :, i, j])
    return y


def _replay(x, packed, geo, tile):
    """The kernel's arithmetic for every workgroup and wave, with the MFMA
    as D[i][j] += sum_k A[i][k] B[k][j], lane l giving A[l%32][l/32] and
    B[l/32][l%32] and holding D rows (r/4)*8 + (l/32)*4 + r%4 of column l%32.
    Pair i's B read is base[step kind of pair i] + offset of k = 2i."""
    N, C, H, W, OC, KH, KW, SH, SW, PT, PL = geo
    TR, TC, OCW = tile
    OH, OW = (H + 2 * PT - KH) // SH + 1, (W + 2 * PL - KW) // SW + 1
    K = C * KH * KW
    npair = (K + 1) // 2
    PR, PC = (TR - 1) * SH + KH, (TC - 1) * SW + KW
    PXG = 4 // OCW
    NB = TR * TC // 32 // PXG
    nblk = packed.shape[0]
    y = np.full((N, OC, OH, OW), np.nan)
    lanes = np.arange(64)
    li, lk = lanes & 31, lanes >> 5
    k0 = 2 * np.arange(npair)
    off = (k0 // (KH * KW) * PR + k0 % (KH * KW) // KW) * PC + k0 % KW
    k1 = k0 + 1
    step = np.where(k1 >= K, 3, np.where(k1 % KW != 0, 0, np.where(k1 % (KH * KW) != 0, 1, 2)))
    delta = np.array([1, PC - KW + 1, (PR - KH + 1) * PC - KW + 1, 0])
    rows = (np.arange(16)[None, :] // 4) * 8 + lk[:, None] * 4 + np.arange(16)[None, :] % 4
    tiles_h, tiles_w = -(-OH // TR), -(-OW // TC)
    for bx in range(N * tiles_h * tiles_w):
        tw, th, n = bx % tiles_w, (bx // tiles_w) % tiles_h, bx // (tiles_w * tiles_h)
        oh0, ow0 = th * TR, tw * TC
        e = np.arange(C * PR * PC)
        c, r, col = e // (PR * PC), (e % (PR * PC)) // PC, e % PC
        ih, iw = oh0 * SH - PT + r, ow0 * SW - PL + col
        ok = (ih >= 0) & (ih < H) & (iw >= 0) & (iw < W)
        patch = np.where(ok, x[n, c, np.clip(ih, 0, H - 1), np.clip(iw, 0, W - 1)], 0.0)
        for by in range(nblk // OCW):
            for wave in range(4):
                ocb, pg = by * OCW + wave % OCW, wave // OCW
                a = packed[ocb].T                                   # [lane][pair]
                for j in range(NB):
                    p = (pg * NB + j) * 32 + li
                    b0 = (p // TC) * SH * PC + (p % TC) * SW
                    idx = b0[:, None] + off[None, :] + lk[:, None] * delta[step][None, :]
                    assert idx.min() >= 0 and idx.max() < patch.size
                    A = np.zeros((npair, 32, 2))
                    B = np.zeros((npair, 2, 32))
                    A[:, li, lk] = a.T
                    B[:, lk, li] = patch[idx].T
                    D = np.einsum("pik,pkj->ij", A, B)
                    oh, ow = oh0 + p // TC, ow0 + p % TC
                    for ln in range(64):
                        if oh[ln] >= OH or ow[ln] >= OW:
                            continue
                        for rr in range(16):
                            oc = ocb * 32 + rows[ln, rr]
                            if oc < OC:
                                y[n, oc, oh[ln], ow[ln]] = D[rows[ln, rr], li[ln]]
    return y


@pytest.mark.parametrize("case", [(1, 3, 23, 21, 64, 7, 2, 3), (1, 3, 17, 19, 32, 3, 2, 1),
                                  (2, 1, 9, 9, 40, 3, 1, 1), (1, 4, 12, 20, 96, 5, 1, 2),
                                  (1, 2, 15, 15, 24, 4, 2, 1)],
                         ids=lambda c: "x".join(map(str, c)))
def test_packed_weights_and_index_replay_match_a_direct_conv(case):
    n, c, h, w, oc, k, s, p = case
    g, feeds = _graph(*case)
    comp = compile_graph(g, feeds=feeds)
    (launch,) = comp.module.plan
    assert launch.kind == "conv_smallc"
    packed = comp.module.device_constants[launch.inputs[1]]
    tile = launch.meta["tile"]
    y = _replay(feeds["x"].astype(np.float64), packed.astype(np.float64),
                (n, c, h, w, oc, k, k, s, s, p, p), tile)
    want = _direct(feeds["x"].astype(np.float64), g.initializers["w"].astype(np.float64), s, p)
    assert not np.isnan(y).any()
    np.testing.assert_allclose(y, want, rtol=1e-10, atol=1e-10)


def test_which_convs_take_the_direct_kernel():
    assert smallc_fits(3, 7, 7, 1, 1) and smallc_pairs(3, 7, 7) == 74
    assert smallc_fits(4, 3, 3, 1, 1)
    assert not smallc_fits(5, 3, 3, 1, 1)           # too many channels
    assert not smallc_fits(3, 3, 3, 2, 2)           # dilated
    assert not smallc_fits(4, 7, 7, 1, 1)           # 98 weight pairs exceed the register budget
    g, feeds = _graph(1, 3, 16, 16, 8, 3, 1, 1)
    kinds = [l.kind for l in compile_graph(g, feeds=feeds, conv_mode="im2col").module.plan]
    assert "conv_smallc" not in kinds
    kinds = [l.kind for l in compile_graph(g, feeds=feeds, small_conv=False, winograd=False).module.plan]
    assert kinds == ["conv"]


def test_tile_rule():
    assert smallc_tile(32, 64, 112, 112) == (8, 16, 2)      # ResNet-18 stem, batch 32
    assert smallc_tile(1, 64, 112, 112) == (4, 16, 2)       # batch 1: more, smaller blocks
    assert smallc_tile(32, 32, 112, 112) == (8, 16, 1)      # MobileNetV2 stem
    assert smallc_tile(64, 256, 16, 16) == (8, 16, 2)
