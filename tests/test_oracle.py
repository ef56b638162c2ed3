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
