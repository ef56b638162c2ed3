"""Pin the NumPy oracle against computations that do not share its code.

The oracle restates mdlc/runtime/ops.py and reference.py; retyping the same
formula would pin nothing, so each function is checked against an
independent route chosen so that a plausible slip (a swapped kh/kw, a wrong
pad side, a dropped bias, a transposed operand, round-half-up instead of
half-even) fails:

* conv / pooling / batchnorm / softmax: torch CPU float64 (F.conv2d,
  max_pool2d, avg_pool2d, batch_norm, softmax) at geometries with stride,
  dilation, asymmetric/SAME padding, groups and ceil_mode;
* im2col: a brute-force Python loop over (c, kh, kw, oh, ow), bitwise;
* gemm: float64 closed form with alpha/beta/transA/transB;
* activations: Python ``math`` per element;
* INT8: Python integers for accumulators, ``fractions``-free float64
  products (exact for 24-bit operands) and Python's round-half-even.

The reference ships no golden-vector files (its tests recompute closed forms
with fixed seeds), so these checks plus the known-answer structure tests in
test_passes.py are what pin the oracle.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops, quant
from oracle.reference import act

torch.set_default_dtype(torch.float64)


def _t(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


CONV_GEOMS = [
    # n, c, h, w, oc, kh, kw, stride, pads(t,l,b,r), dil, group
    (1, 3, 9, 9, 8, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 1),
    (2, 4, 10, 7, 6, 3, 2, (2, 1), (1, 0, 2, 1), (1, 2), 1),
    (2, 6, 8, 8, 6, 3, 3, (1, 1), (1, 1, 1, 1), (1, 1), 6),     # depthwise
    (1, 4, 9, 9, 8, 3, 3, (2, 2), (0, 0, 0, 0), (1, 1), 2),     # grouped
    (3, 2, 11, 11, 5, 7, 7, (2, 2), (3, 3, 3, 3), (1, 1), 1),
]


@pytest.mark.parametrize("geom", CONV_GEOMS)
def test_conv_matches_torch_float64(geom):
    n, c, h, w, oc, kh, kw, st, pads, dil, group = geom
    rng = np.random.default_rng(21)
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    wt = rng.standard_normal((oc, c // group, kh, kw)).astype(np.float32)
    b = rng.standard_normal(oc).astype(np.float32)
    pt, pl, pb, pr = pads
    got = ops.conv(x, wt, b, strides=list(st), pads=[pt, pl, pb, pr], dilations=list(dil),
                   group=group)
    xp = F.pad(_t(x), (pl, pr, pt, pb))
    want = F.conv2d(xp, _t(wt), _t(b), stride=st, dilation=dil, groups=group).numpy()
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_conv_same_upper_and_lower_padding():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 2, 8, 8)).astype(np.float32)
    wt = rng.standard_normal((3, 2, 4, 4)).astype(np.float32)
    for mode, (lo, hi) in (("SAME_UPPER", (1, 2)), ("SAME_LOWER", (2, 1))):
        got = ops.conv(x, wt, None, strides=[1, 1], pads=None, dilations=[1, 1], group=1,
                       auto_pad=mode)
        want = F.conv2d(F.pad(_t(x), (lo, hi, lo, hi)), _t(wt)).numpy()
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
        assert got.shape == (1, 3, 8, 8)


def test_im2col_bitwise_against_brute_force():
    rng = np.random.default_rng(1)
    n, c, h, w, kh, kw, sh, sw, dh, dw = 2, 3, 6, 7, 3, 2, 2, 1, 1, 2
    pads = ((1, 0), (2, 1))
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    cols, oh, ow = ops.im2col(x, kh, kw, sh, sw, dh, dw, pads)
    for b in range(n):
        for ci in range(c):
            for i in range(kh):
                for j in range(kw):
                    r = (ci * kh + i) * kw + j
                    for y in range(oh):
                        for z in range(ow):
                            yy = y * sh - pads[0][0] + i * dh
                            zz = z * sw - pads[1][0] + j * dw
                            v = x[b, ci, yy, zz] if 0 <= yy < h and 0 <= zz < w else 0.0
                            assert cols[b, r, y * ow + z] == v


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_closed_form(ta, tb):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((5, 7) if not ta else (7, 5)).astype(np.float32)
    b = rng.standard_normal((7, 4) if not tb else (4, 7)).astype(np.float32)
    c = rng.standard_normal(4).astype(np.float32)
    got = ops.gemm(a, b, c, alpha=0.5, beta=2.0, transA=ta, transB=tb)
    A = a.astype(np.float64).T if ta else a.astype(np.float64)
    B = b.astype(np.float64).T if tb else b.astype(np.float64)
    want = np.array([[0.5 * sum(A[i, k] * B[k, j] for k in range(7)) + 2.0 * c[j]
                      for j in range(4)] for i in range(5)])
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("ceil", [0, 1])
def test_maxpool_matches_torch(ceil):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 11, 11)).astype(np.float32)
    got = ops.maxpool(x, kernel=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1], ceil_mode=ceil)
    want = F.max_pool2d(_t(x), 3, 2, padding=1, ceil_mode=bool(ceil)).numpy()
    np.testing.assert_array_equal(got, want.astype(np.float32))


def test_maxpool_ceil_mode_partial_window_is_a_reference_limitation():
    """With ceil_mode=1 and a last window that hangs past the padded input,
    the reference's strided-slice formulation (ops.py:119-124) yields a
    shorter slice and NumPy raises; the oracle keeps that behaviour, so such
    shapes have no oracle (the device kernel bounds-checks every tap)."""
    x = np.zeros((1, 1, 10, 10), np.float32)
    with pytest.raises(ValueError):
        ops.maxpool(x, kernel=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1], ceil_mode=1)


@pytest.mark.parametrize("cip", [0, 1])
def test_averagepool_matches_torch(cip):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1, 2, 9, 9)).astype(np.float32)
    got = ops.averagepool(x, kernel=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1],
                          count_include_pad=cip)
    want = F.avg_pool2d(_t(x), 3, 2, padding=1, count_include_pad=bool(cip)).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)


def test_global_average_pool_and_batchnorm_and_softmax():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 4, 7, 7)).astype(np.float32)
    np.testing.assert_allclose(ops.global_average_pool(x),
                               _t(x).mean(dim=(2, 3), keepdim=True).numpy(), rtol=1e-6, atol=1e-7)
    s, b, m = (rng.standard_normal(4).astype(np.float32) for _ in range(3))
    v = rng.uniform(0.5, 1.5, 4).astype(np.float32)
    want = F.batch_norm(_t(x), _t(m), _t(v), _t(s), _t(b), training=False, eps=1e-5).numpy()
    np.testing.assert_allclose(ops.batchnorm(x, s, b, m, v), want, rtol=1e-5, atol=1e-6)
    z = rng.standard_normal((3, 9)).astype(np.float32)
    np.testing.assert_allclose(ops.softmax(z, axis=1), torch.softmax(_t(z), 1).numpy(),
                               rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name,attrs,fn", [
    ("Relu", {}, lambda v: max(v, 0.0)),
    ("Clip", {"clip_min": 0.0, "clip_max": 6.0}, lambda v: min(max(v, 0.0), 6.0)),
    ("Sigmoid", {}, lambda v: 1.0 / (1.0 + math.exp(-v))),
    ("Tanh", {}, math.tanh),
    ("LeakyRelu", {"alpha": 0.1}, lambda v: v if v >= 0 else 0.1 * v),
    ("HardSigmoid", {"alpha": 0.2, "beta": 0.5}, lambda v: min(max(0.2 * v + 0.5, 0.0), 1.0)),
    ("HardSwish", {}, lambda v: v * min(max(v / 6.0 + 0.5, 0.0), 1.0)),
])
def test_activations_closed_form(name, attrs, fn):
    x = np.linspace(-8, 8, 161).astype(np.float32)
    got = act(name, x, attrs)
    want = np.array([fn(float(v)) for v in x])
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-7)


# ----- INT8 semantics ---------------------------------------------------------

def test_requant_rounds_half_to_even_and_clamps():
    acc = np.array([1, 3, 5, -5, -3, 254, 255, 1000, -1000, 0], dtype=np.int32)
    got = quant.requant(acc, np.float32(0.5))
    want = [max(-127, min(127, round(float(np.float32(a) * np.float32(0.5))))) for a in acc]
    assert got.tolist() == want                # Python round() is half-to-even
    assert got[:5].tolist() == [0, 2, 2, -2, -2]
    assert quant.requant(acc, np.float32(0.5), lo=0).min() == 0


def test_requant_matches_float64_route():
    """float32(acc)*m rounded once == float64 product of the two float32
    values rounded to float32 (exact: 24x24-bit products fit in 53 bits)."""
    rng = np.random.default_rng(8)
    acc = rng.integers(-2**27, 2**27, 20000).astype(np.int32)
    m = rng.uniform(1e-6, 1e-2, 20000).astype(np.float32)
    got = quant.requant(acc, m)
    prod = (np.float64(1) * acc.astype(np.float32).astype(np.float64) * m.astype(np.float64))
    f32 = prod.astype(np.float32)
    want = np.array([max(-127, min(127, round(float(v)))) for v in f32], dtype=np.int8)
    np.testing.assert_array_equal(got, want)


def test_int8_conv_and_gemm_accumulators_exact():
    rng = np.random.default_rng(9)
    x = rng.integers(-127, 128, (2, 4, 6, 6)).astype(np.int8)
    w = rng.integers(-127, 128, (6, 2, 3, 3)).astype(np.int8)
    b = rng.integers(-5000, 5000, 6).astype(np.int32)
    acc = quant.conv_acc(x, w, b, strides=[2, 1], pads=[1, 1, 1, 1], dilations=[1, 1], group=2)
    want = F.conv2d(F.pad(_t(x), (1, 1, 1, 1)), _t(w), _t(b), stride=(2, 1), groups=2).numpy()
    np.testing.assert_array_equal(acc, want.astype(np.int64))
    xa = rng.integers(-127, 128, (3, 5)).astype(np.int8)
    wt = rng.integers(-127, 128, (4, 5)).astype(np.int8)
    bb = rng.integers(-100, 100, 4).astype(np.int32)
    g = quant.gemm_acc(xa, wt, bb)
    want = [[sum(int(xa[i, k]) * int(wt[j, k]) for k in range(5)) + int(bb[j]) for j in range(4)]
            for i in range(3)]
    assert g.tolist() == want


def test_qadd_lut_quantize_dequantize():
    a = np.array([10, -20, 127, -127], np.int8)
    b = np.array([5, 5, 127, -127], np.int8)
    got = quant.qadd(a, b, np.float32(0.5), np.float32(0.25))
    want = [max(-127, min(127, round(float(np.float32(np.float32(x) * np.float32(0.5))
                                           + np.float32(np.float32(y) * np.float32(0.25))))))
            for x, y in zip(a, b)]
    assert got.tolist() == want
    table = np.arange(-128, 128)[::-1].clip(-127, 127).astype(np.int8)
    assert quant.lut(a, table).tolist() == [int(table[int(v) + 128]) for v in a]
    q = quant.quantize(np.array([0.05, 0.15, -0.25, 100.0], np.float32), np.float32(10.0))
    assert q.tolist() == [0, 2, -2, 127]
    assert quant.dequantize(np.array([3], np.int8), 0.5).tolist() == [1.5]


def test_a_planted_im2col_slip_is_caught(monkeypatch):
    """Swap kh/kw in the oracle's im2col: the torch conv check must fail."""
    real = ops.im2col

    def slipped(x, kh, kw, sh, sw, dh, dw, pads):
        cols, oh, ow = real(x, kh, kw, sh, sw, dh, dw, pads)
        n, k, p = cols.shape
        c = k // (kh * kw)
        return cols.reshape(n, c, kh, kw, p).transpose(0, 1, 3, 2, 4).reshape(n, k, p), oh, ow

    monkeypatch.setattr(ops, "im2col", slipped)
    with pytest.raises(AssertionError):
        test_conv_matches_torch_float64(CONV_GEOMS[0])


# ----- quantized global average pool (RepViT's head) ------------------------------

def _qgap_brute(q, mult, flatten):
    """Python-integer sum over each plane, one float32 multiply (float64
    product of two float32 values is exact, then rounded once), Python's
    round-half-even, clamp to [-127, 127]."""
    n, c, h, w = q.shape
    m = float(np.float32(mult))
    out = []
    for i in range(n):
        row = []
        for j in range(c):
            s = sum(int(q[i, j, y, x]) for y in range(h) for x in range(w))
            f = float(np.float32(float(np.float32(s)) * m))
            row.append(max(-127, min(127, round(f))))
        out.append(row if flatten else [[[v]] for v in row])
    return np.array(out, dtype=np.int64)


def _qgap_graph(shape, mult, flatten):
    from mdlc_amd.ir import Graph, Node

    g = Graph("qgap")
    g.inputs, g.outputs = ["q"], ["y"]
    g.add_node(Node("QGlobalAveragePool", ["q"], ["y"], {"mult": np.float32(mult), "flatten": flatten}))
    return g


@pytest.mark.parametrize("flatten", [False, True])
def test_qgap_matches_integer_brute_force(flatten):
    from oracle.reference import run_reference

    rng = np.random.default_rng(21)
    # 7x7 planes of codes, and a multiplier that puts ties (x.5) and values
    # beyond +-127 among the results
    q = rng.integers(-127, 128, (2, 6, 7, 7)).astype(np.int8)
    q[0, 0] = 127                                   # sum 6223 -> saturates high
    q[1, 1] = -127                                  # saturates low
    q[0, 2] = 0
    q[0, 2, 0, :3] = (1, 2, 2)                      # sum 5: 2.5 -> 2 (half to even)
    q[0, 3] = 0
    q[0, 3, 0, :2] = (3, 4)                         # sum 7: 3.5 -> 4
    mult = 0.5
    got = run_reference(_qgap_graph(q.shape, mult, flatten), {"q": q})["y"]
    want = _qgap_brute(q, mult, flatten)
    assert got.dtype == np.int8 and got.shape == want.shape
    np.testing.assert_array_equal(got.astype(np.int64), want)
    flat = want.reshape(2, 6)
    assert flat[0, 0] == 127 and flat[1, 1] == -127 and flat[0, 2] == 2 and flat[0, 3] == 4
    # the RepViT multiplier form s_in / (HW * s_out)
    mult = np.float32(0.05 / (49 * 0.03))
    np.testing.assert_array_equal(quant.global_avg_pool(q, mult).astype(np.int64),
                                  _qgap_brute(q, mult, False))


def test_qgap_planted_slips_are_caught(monkeypatch):
    """Half-up rounding, or a sum over the wrong axes, must fail the check."""
    real_rint = np.rint
    monkeypatch.setattr(quant.np, "rint", lambda x: np.floor(np.asarray(x) + 0.5))
    with pytest.raises(AssertionError):
        test_qgap_matches_integer_brute_force(False)
    monkeypatch.setattr(quant.np, "rint", real_rint)

    real_gap = quant.global_avg_pool

    def wrong_axes(q, mult):                        # sums the rows of one column only
        acc = q.astype(np.int64).sum(axis=2, keepdims=True)[:, :, :, :1]
        return quant.requant(acc.astype(np.int32), mult)

    monkeypatch.setattr(quant, "global_avg_pool", wrong_axes)
    with pytest.raises(AssertionError):
        test_qgap_matches_integer_brute_force(False)
    monkeypatch.setattr(quant, "global_avg_pool", real_gap)


# ----- views, pad and matmul ------------------------------------------------------

def _fill_c_order(values, shape):
    """Place ``values`` (a flat list) into ``shape`` one index at a time in
    row-major order, without NumPy's reshape."""
    out = np.empty(shape, dtype=np.float64)
    for k, idx in enumerate(np.ndindex(*shape)):
        out[idx] = values[k]
    return out


@pytest.mark.parametrize("shape,axis", [((2, 3, 4, 5), 1), ((2, 3, 4, 5), 0), ((2, 3, 4, 5), 3),
                                        ((2, 3, 4, 5), -2), ((6, 1, 1), 1), ((4,), 1)])
def test_flatten_closed_form(shape, axis):
    x = np.arange(int(np.prod(shape)), dtype=np.float32).reshape(shape) * 0.5 - 3
    k = axis + len(shape) if axis < 0 else axis
    lead = 1
    for d in shape[:k]:
        lead *= d
    want_shape = (lead, int(np.prod(shape)) // lead)
    got = ops.flatten(x, axis)
    flat = [float(x[idx]) for idx in np.ndindex(*shape)]
    assert got.shape == want_shape
    np.testing.assert_array_equal(got, _fill_c_order(flat, want_shape))


@pytest.mark.parametrize("shape,target,want_shape", [
    ((2, 3, 4), [0, -1], (2, 12)),          # 0 copies the input dim
    ((2, 3, 4), [4, 0, 2], (4, 3, 2)),
    ((2, 3, 4), [-1], (24,)),
    ((2, 512, 1, 1), [0, 512], (2, 512)),
    ((6, 4), [2, 3, 4], (2, 3, 4)),
])
def test_reshape_closed_form(shape, target, want_shape):
    x = np.arange(int(np.prod(shape)), dtype=np.float32).reshape(shape) - 7
    got = ops.reshape(x, np.array(target, dtype=np.int64))
    flat = [float(x[idx]) for idx in np.ndindex(*shape)]
    assert got.shape == want_shape
    np.testing.assert_array_equal(got, _fill_c_order(flat, want_shape))


def _pad_brute(x, pads, value, mode):
    half = len(pads) // 2
    before, after = pads[:half], pads[half:]
    out_shape = tuple(s + b + a for s, b, a in zip(x.shape, before, after))
    out = np.empty(out_shape, dtype=np.float64)
    for idx in np.ndindex(*out_shape):
        src, inside = [], True
        for d, i in enumerate(idx):
            j, n = i - before[d], x.shape[d]
            if 0 <= j < n:
                src.append(j)
            elif mode == "constant":
                inside = False
                break
            elif mode == "edge":
                src.append(min(max(j, 0), n - 1))
            else:                                   # reflect: mirror without repeating the edge
                period = 2 * (n - 1)
                j = abs(j) % period
                src.append(period - j if j >= n else j)
        out[idx] = float(x[tuple(src)]) if inside else value
    return out


@pytest.mark.parametrize("mode,value", [("constant", 0.0), ("constant", -2.5), ("edge", 0.0),
                                        ("reflect", 0.0)])
def test_pad_brute_force(mode, value):
    rng = np.random.default_rng(31)
    x = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    pads = [0, 1, 2, 0, 0, 0, 1, 3]                 # begins then ends, per axis
    got = ops.pad(x, np.array(pads), value, mode)
    np.testing.assert_array_equal(got.astype(np.float64), _pad_brute(x, pads, value, mode))


@pytest.mark.parametrize("a_shape,b_shape", [((5, 7), (7, 3)), ((2, 5, 7), (7, 3)),
                                             ((2, 5, 7), (2, 7, 3)), ((1, 9), (9, 1))])
def test_matmul_brute_force(a_shape, b_shape):
    rng = np.random.default_rng(41)
    a = rng.standard_normal(a_shape).astype(np.float32)
    b = rng.standard_normal(b_shape).astype(np.float32)
    got = ops.matmul(a, b)
    A = a.reshape((-1,) + a_shape[-2:]).astype(np.float64)
    B = np.broadcast_to(b, a_shape[:-2] + b_shape[-2:]).reshape((-1,) + b_shape[-2:]).astype(np.float64)
    want = np.zeros((A.shape[0], a_shape[-2], b_shape[-1]))
    for n in range(A.shape[0]):
        for i in range(a_shape[-2]):
            for j in range(b_shape[-1]):
                want[n, i, j] = sum(A[n, i, k] * B[n, k, j] for k in range(a_shape[-1]))
    assert got.shape == a_shape[:-1] + b_shape[-1:]
    np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-5, atol=1e-5)


def test_view_and_matmul_planted_slips_are_caught(monkeypatch):
    monkeypatch.setattr(ops, "matmul", lambda a, b: a @ b[..., ::-1])   # columns out of order
    with pytest.raises(AssertionError):
        test_matmul_brute_force((5, 7), (7, 3))
    monkeypatch.undo()
    monkeypatch.setattr(ops, "flatten", lambda x, axis=1: x.transpose().reshape(
        int(np.prod(x.shape[:axis])) if axis > 0 else 1, -1))
    with pytest.raises(AssertionError):
        test_flatten_closed_form((2, 3, 4, 5), 1)
    monkeypatch.undo()
    real_pad = ops.pad
    monkeypatch.setattr(ops, "pad", lambda x, pads, value=0.0, mode="constant":
                        real_pad(x, np.roll(np.asarray(pads), len(pads) // 2), value, mode))
    with pytest.raises(AssertionError):
        test_pad_brute_force("constant", -2.5)


def test_float64_group_rerun_matches_torch_float64():
    """``run_groups_float64`` on the stated-weights ResNet-18 (a 56x56 input
    keeps it small): every folded conv group equals torch's float64 conv2d +
    bias + ReLU (+ the residual add) on the widened float32 inputs to float64
    rounding, and differs from the float32 oracle by float32 rounding. A
    planted slip that re-runs the groups without widening their inputs (so
    every sum rounds to float32) is caught by the same comparison."""
    from mdlc_amd.compiler import compile_graph
    from mdlc_amd.tools.build_resnet18 import build_resnet18
    from oracle import reference
    from oracle.reference import run_groups_float64, run_reference

    g = build_resnet18(batch=1)
    x = np.random.default_rng(3).standard_normal((1, 3, 224, 224)).astype(np.float32)
    c = compile_graph(g, feeds={"input": x})
    env32 = run_reference(c.graph, {"input": x}, return_all=True)
    want64 = run_groups_float64(c.graph, env32)

    def torch_group(n, env):
        t = lambda e: torch.from_numpy(np.asarray(env[e], np.float64))  # noqa: E731
        a = n.attrs
        p = a["pads"]
        y = F.conv2d(F.pad(t(n.inputs[0]), (p[1], p[3], p[0], p[2])), t(n.inputs[1]),
                     t(n.inputs[2]) if len(n.inputs) > 2 and n.inputs[2] else None,
                     stride=a["strides"], dilation=a.get("dilations", [1, 1]))
        if a.get("residual_subgraph"):
            if a.get("activation") == "Relu":
                y = torch.relu(y)
            y = torch.relu(y + t(n.inputs[3]))
        elif a.get("activation") == "Relu":
            y = torch.relu(y)
        return y.numpy()

    convs = [n for n in c.graph.nodes if n.op_type in ("FusedConvAct", "Conv") and len(n.inputs) >= 2]
    assert len(convs) >= 15
    for n in convs:
        ref = torch_group(n, env32)
        o = n.outputs[0]
        assert want64[o].dtype == np.float64
        np.testing.assert_allclose(want64[o], ref, rtol=1e-12, atol=1e-12)
        assert 0 < np.abs(env32[o] - want64[o]).max() < 1e-4 * max(1.0, np.abs(ref).max())

    # planted: the re-run forgets to widen, so it is the float32 oracle again
    def slipped(graph, env):
        ex = reference.ReferenceExecutor(graph)
        return {n.outputs[0]: ex.exec_node(n, env)[0] for n in graph.nodes}

    bad = slipped(c.graph, env32)
    n = convs[-1]
    assert not np.allclose(bad[n.outputs[0]], torch_group(n, env32), rtol=1e-12, atol=1e-12)


def test_check_against_float64_rule():
    """The float64-relative bar: a float32 result as accurate as the float32
    reference passes at either magnitude; one with a dropped term fails."""
    from mdlc_amd.testing import DEVICE_TENSOR, check_against_float64

    rng = np.random.default_rng(0)
    for scale in (1.0, 300.0):
        a = rng.standard_normal((64, 2304)) * scale
        b = rng.standard_normal((2304, 49))
        want64 = a @ b
        ref32 = (a.astype(np.float32) @ b.astype(np.float32)).astype(np.float32)
        # the same sums in another float32 order (blocked, like a tiled kernel)
        dev = sum((a[:, k:k + 64].astype(np.float32) @ b[k:k + 64].astype(np.float32))
                  for k in range(0, 2304, 64)).astype(np.float32)
        r = check_against_float64("x", dev, ref32, want64, rtol=DEVICE_TENSOR.rtol,
                                  atol=DEVICE_TENSOR.atol)
        assert r.ok, r
        dropped = dev - (a[:, :1].astype(np.float32) @ b[:1].astype(np.float32))
        r = check_against_float64("x", dropped, ref32, want64, rtol=DEVICE_TENSOR.rtol,
                                  atol=DEVICE_TENSOR.atol)
        assert not r.ok and r.device > 10 * r.bound, r
