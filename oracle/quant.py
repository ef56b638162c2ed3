"""INT8 quantized op semantics — oracle definition (test infrastructure only).

The reference has no quantized operator: ``DType.INT8`` exists
(mdlc/ir/tensor.py:20-22,29,37) but its executor raises on anything it does
not know (mdlc/runtime/reference.py:184). The semantics below are therefore
defined by this build and are the contract the HIP kernels must meet
bit-for-bit:

* Symmetric int8, zero point 0, codes clamped to [-127, 127].
* Integer products accumulate exactly in int32 (checked against int64).
* Requantization: ``q = clamp(rint(float32(acc) * m), lo, 127)`` where
  ``float32(acc)`` is round-to-nearest-even, ``m`` is a float32 multiplier
  (per output channel or per tensor), the product is one correctly rounded
  float32 multiply (no fused multiply-add), ``rint`` rounds half to even, and
  ``lo`` is 0 after a fused ReLU, else -127.
* Quantize: ``q = clamp(rint(x * inv_s), -127, 127)`` with ``inv_s`` a float32.
* Residual add: ``clamp(rint(f32(f32(a)*ma) + f32(f32(b)*mb)), -127, 127)``,
  each step a separately rounded float32 operation.
* Lookup (e.g. GELU): ``table[q + 128]`` with a 256-entry int8 table.
* Dequantize: ``float32(q) * s`` (one float32 multiply).
"""

from __future__ import annotations

import numpy as np

QMIN, QMAX = -127, 127


def requant(acc, mult, lo: int = QMIN):
    """acc int32 array, mult float32 broadcastable → int8."""
    f = acc.astype(np.float32) * np.asarray(mult, dtype=np.float32)
    return np.clip(np.rint(f), lo, QMAX).astype(np.int8)


def quantize(x, inv_scale):
    f = np.asarray(x, dtype=np.float32) * np.float32(inv_scale)
    return np.clip(np.rint(f), QMIN, QMAX).astype(np.int8)


def dequantize(q, scale):
    return q.astype(np.float32) * np.float32(scale)


def conv_acc(x, w, bias, *, strides, pads, dilations, group):
    """Exact int32 accumulator of an int8 conv (zero padding), + int32 bias.

    Computed as an int64 einsum over an im2col matrix, then checked to fit
    int32 and narrowed.
    """
    from oracle.ops import im2col, resolve_pads

    n, c, ih, iw = x.shape
    oc, icg, kh, kw = w.shape
    sh, sw = strides
    dh, dw = dilations
    p = resolve_pads("NOTSET", pads, (ih, iw), (kh, kw), (sh, sw), (dh, dw))
    x64 = x.astype(np.int64)
    w64 = w.astype(np.int64)
    ocg = oc // group
    parts = []
    for g in range(group):
        cols, oh, ow = im2col(x64[:, g * icg:(g + 1) * icg], kh, kw, sh, sw, dh, dw, p)
        wg = w64[g * ocg:(g + 1) * ocg].reshape(ocg, -1)
        parts.append(np.einsum("ok,nkp->nop", wg, cols).reshape(n, ocg, oh, ow))
    acc = np.concatenate(parts, axis=1)
    if bias is not None:
        acc = acc + bias.astype(np.int64).reshape(1, -1, 1, 1)
    assert np.abs(acc).max(initial=0) < 2**31, "int32 accumulator overflow"
    return acc.astype(np.int32)


def gemm_acc(x, w_t, bias):
    """x int8 [M,K], w_t int8 [N,K] (transB layout) → exact int32 [M,N] + bias."""
    acc = x.astype(np.int64) @ w_t.astype(np.int64).T
    if bias is not None:
        acc = acc + bias.astype(np.int64)[None, :]
    assert np.abs(acc).max(initial=0) < 2**31, "int32 accumulator overflow"
    return acc.astype(np.int32)


def qadd(a, b, ma, mb):
    t1 = a.astype(np.float32) * np.float32(ma)
    t2 = b.astype(np.float32) * np.float32(mb)
    return np.clip(np.rint(t1 + t2), QMIN, QMAX).astype(np.int8)


def lut(q, table):
    return np.asarray(table, dtype=np.int8)[q.astype(np.int16) + 128]


def global_avg_pool(q, mult):
    """Sum over H,W in int32, then requantize with ``mult`` (= s_in/(HW*s_out))."""
    acc = q.astype(np.int64).sum(axis=(2, 3), keepdims=True)
    return requant(acc.astype(np.int32), mult)
