"""NumPy op semantics — oracle restatement of mdlc/runtime/ops.py.

Test infrastructure only (see ``oracle/__init__.py``). Each function names the
reference lines it restates; the arithmetic calls are the same NumPy calls so
float32 results match the reference's.
"""

from __future__ import annotations

import numpy as np


def resolve_pads(auto_pad, pads, in_hw, k_hw, s_hw, d_hw):
    """ops.py:15-32 — ((top, bottom), (left, right))."""
    if auto_pad in ("SAME_UPPER", "SAME_LOWER"):
        out = []
        for i, k, s, d in zip(in_hw, k_hw, s_hw, d_hw):
            o = -(-i // s)
            tot = max(0, (o - 1) * s + (k - 1) * d + 1 - i)
            lo, hi = tot // 2, tot - tot // 2
            out.append((lo, hi) if auto_pad == "SAME_UPPER" else (hi, lo))
        return tuple(out)
    if pads is None:
        return (0, 0), (0, 0)
    return (pads[0], pads[2]), (pads[1], pads[3])


def im2col(x, kh, kw, sh, sw, dh, dw, pads):
    """ops.py:35-51 — (N, C*kh*kw, OH*OW), row index (c, ky, kx) with kx fastest."""
    n, c, h, w = x.shape
    (pt, pb), (pl, pr) = pads
    xp = np.pad(x, ((0, 0), (0, 0), (pt, pb), (pl, pr)))
    oh = (h + pt + pb - (dh * (kh - 1) + 1)) // sh + 1
    ow = (w + pl + pr - (dw * (kw - 1) + 1)) // sw + 1
    cols = np.empty((n, c * kh * kw, oh * ow), dtype=x.dtype)
    r = 0
    for ci in range(c):
        for ky in range(kh):
            for kx in range(kw):
                win = xp[:, ci, ky * dh: ky * dh + sh * oh: sh, kx * dw: kx * dw + sw * ow: sw]
                cols[:, r, :] = win.reshape(n, oh * ow)
                r += 1
    return cols, oh, ow


def conv(x, w, b, *, strides, pads, dilations, group, auto_pad="NOTSET"):
    """ops.py:56-81 — im2col + ``np.einsum("ok,nkp->nop")`` per group, + bias."""
    n, c, ih, iw = x.shape
    oc, icg, kh, kw = w.shape
    sh, sw = strides
    dh, dw = dilations
    p = resolve_pads(auto_pad, pads, (ih, iw), (kh, kw), (sh, sw), (dh, dw))
    if group == 1:
        cols, oh, ow = im2col(x, kh, kw, sh, sw, dh, dw, p)
        y = np.einsum("ok,nkp->nop", w.reshape(oc, -1), cols).reshape(n, oc, oh, ow)
    else:
        ocg = oc // group
        parts = []
        for g in range(group):
            cols, oh, ow = im2col(x[:, g * icg:(g + 1) * icg], kh, kw, sh, sw, dh, dw, p)
            wg = w[g * ocg:(g + 1) * ocg].reshape(ocg, -1)
            parts.append(np.einsum("ok,nkp->nop", wg, cols).reshape(n, ocg, oh, ow))
        y = np.concatenate(parts, axis=1)
    if b is not None:
        y = y + b.reshape(1, -1, 1, 1)
    return y


def gemm(a, b, c, *, alpha=1.0, beta=1.0, transA=0, transB=0):
    """ops.py:84-92 — alpha*(a@b) + beta*c."""
    if transA:
        a = a.T
    if transB:
        b = b.T
    y = alpha * (a @ b)
    if c is not None:
        y = y + beta * c
    return y


def matmul(a, b):
    """ops.py:95-96."""
    return a @ b


def batchnorm(x, scale, bias, mean, var, *, epsilon=1e-5):
    """ops.py:99-106."""
    shp = [1] * x.ndim
    shp[1] = x.shape[1]
    return (x - mean.reshape(shp)) / np.sqrt(var.reshape(shp) + epsilon) * scale.reshape(shp) \
        + bias.reshape(shp)


def maxpool(x, *, kernel, strides, pads, dilations=(1, 1), auto_pad="NOTSET", ceil_mode=0):
    """ops.py:109-125 — -inf padding, window max over strided slices."""
    n, c, ih, iw = x.shape
    kh, kw = kernel
    sh, sw = strides
    dh, dw = dilations
    (pt, pb), (pl, pr) = resolve_pads(auto_pad, pads, (ih, iw), (kh, kw), (sh, sw), (dh, dw))
    xp = np.pad(x, ((0, 0), (0, 0), (pt, pb), (pl, pr)), constant_values=-np.inf)
    q = (lambda a, d: -(-a // d)) if ceil_mode else (lambda a, d: a // d)
    oh = q(ih + pt + pb - (dh * (kh - 1) + 1), sh) + 1
    ow = q(iw + pl + pr - (dw * (kw - 1) + 1), sw) + 1
    y = np.full((n, c, oh, ow), -np.inf, dtype=x.dtype)
    for ky in range(kh):
        for kx in range(kw):
            win = xp[:, :, ky * dh: ky * dh + sh * oh: sh, kx * dw: kx * dw + sw * ow: sw]
            y = np.maximum(y, win[:, :, :oh, :ow])
    return y


def averagepool(x, *, kernel, strides, pads, auto_pad="NOTSET", count_include_pad=0, ceil_mode=0):
    """ops.py:128-146 — float64 accumulation, divide by window or valid count."""
    n, c, ih, iw = x.shape
    kh, kw = kernel
    sh, sw = strides
    (pt, pb), (pl, pr) = resolve_pads(auto_pad, pads, (ih, iw), (kh, kw), (sh, sw), (1, 1))
    xp = np.pad(x, ((0, 0), (0, 0), (pt, pb), (pl, pr)))
    q = (lambda a, d: -(-a // d)) if ceil_mode else (lambda a, d: a // d)
    oh = q(ih + pt + pb - kh, sh) + 1
    ow = q(iw + pl + pr - kw, sw) + 1
    acc = np.zeros((n, c, oh, ow), dtype=np.float64)
    cnt = np.zeros((n, c, oh, ow), dtype=np.float64)
    ones = np.pad(np.ones((n, c, ih, iw)), ((0, 0), (0, 0), (pt, pb), (pl, pr)))
    for ky in range(kh):
        for kx in range(kw):
            acc += xp[:, :, ky: ky + sh * oh: sh, kx: kx + sw * ow: sw][:, :, :oh, :ow]
            cnt += ones[:, :, ky: ky + sh * oh: sh, kx: kx + sw * ow: sw][:, :, :oh, :ow]
    den = (kh * kw) if count_include_pad else np.maximum(cnt, 1)
    return (acc / den).astype(x.dtype)


def global_average_pool(x):
    """ops.py:149-150."""
    return x.mean(axis=tuple(range(2, x.ndim)), keepdims=True).astype(x.dtype)


def relu(x):
    return np.maximum(x, 0)                       # ops.py:155-156


def clip(x, lo=None, hi=None):
    lo = -np.inf if lo is None else lo            # ops.py:159-164
    hi = np.inf if hi is None else hi
    return np.clip(x, lo, hi)


def leaky_relu(x, alpha=0.01):
    return np.where(x >= 0, x, alpha * x)         # ops.py:167-168


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))               # ops.py:171-172


def tanh(x):
    return np.tanh(x)                             # ops.py:175-176


def hard_sigmoid(x, alpha=0.2, beta=0.5):
    return np.clip(alpha * x + beta, 0.0, 1.0)    # ops.py:179-180


def hard_swish(x):
    return x * np.clip(x / 6.0 + 0.5, 0.0, 1.0)   # ops.py:183-185


def softmax(x, axis=-1):
    z = x - np.max(x, axis=axis, keepdims=True)   # ops.py:188-191
    e = np.exp(z)
    return e / np.sum(e, axis=axis, keepdims=True)


def flatten(x, axis=1):
    axis = axis + x.ndim if axis < 0 else axis    # ops.py:213-217
    lead = int(np.prod(x.shape[:axis])) if axis > 0 else 1
    return x.reshape(lead, -1)


def reshape(x, shape):
    tgt = [int(s) for s in np.asarray(shape).ravel()]   # ops.py:220-226
    return x.reshape([x.shape[i] if s == 0 else s for i, s in enumerate(tgt)])


def pad(x, pads, value=0.0, mode="constant"):
    p = [int(v) for v in np.asarray(pads).ravel()]      # ops.py:249-255
    half = len(p) // 2
    width = [(p[i], p[i + half]) for i in range(half)]
    if mode == "constant":
        return np.pad(x, width, mode="constant", constant_values=value)
    return np.pad(x, width, mode={"reflect": "reflect", "edge": "edge"}.get(mode, "constant"))
