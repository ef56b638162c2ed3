"""RepViT-style INT8 model built straight into the IR (benchmark config 4).

The reference exports timm's ``repvit_m0_9`` (mdlc/tools/build_repvit.py:
25-57) but has no quantized path; this builder writes the quantized
deploy-form network directly, with the structure and distributions the
benchmark config names:

* input fp32 [N,3,224,224] -> QuantizeLinear;
* stem: 3x3 s2 conv 3->24, GELU, 3x3 s2 conv 24->48 (to 56x56);
* four stages of widths 48/96/192/384 and depths 3/3/15/2; each block is a
  re-parameterised depthwise 3x3 token mixer followed by a residual channel
  mixer 1x1 C->2C, GELU, 1x1 2C->C, added back with a quantized Add; the
  first block of stages 2-4 first downsamples with a depthwise 3x3 stride-2
  conv and a 1x1 conv to the new width;
* global average pool, flatten, and a 384->1000 classifier whose int32
  accumulators are dequantized to float32 logits.

Quantization: weights symmetric per output channel, w ~ N(0, 0.05),
s_w = max|w|/127, q_w = rint(w/s_w); every activation tensor gets a per-tensor
scale drawn from U(0.01, 0.1); biases are int32, b ~ N(0, 0.1) quantized with
s_x*s_w. A conv's output codes are clamp(rint(float32(acc) * m), lo, 127)
with m = float32(s_x*s_w[oc]/s_y) (lo = -127, or 0 after a fused ReLU). GELU
(tanh form) is a 256-entry int8->int8 table from the input to the output
scale. Operator semantics are defined in ``oracle/quant.py``.
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import DType, Graph
from mdlc_amd.tools.graph_builder import GraphBuilder

WIDTHS = (48, 96, 192, 384)
DEPTHS = (3, 3, 15, 2)


def gelu_tanh(v: np.ndarray) -> np.ndarray:
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


def gelu_table(s_in: float, s_out: float) -> np.ndarray:
    codes = np.arange(-128, 128, dtype=np.float64)
    y = gelu_tanh(codes * s_in) / s_out
    return np.clip(np.rint(y), -127, 127).astype(np.int8)


class _QBuilder:
    def __init__(self, name: str, seed: int) -> None:
        self.b = GraphBuilder(name, seed)
        self.rng = self.b.rng
        self.scale: dict = {}
        self.k = 0

    def new_scale(self) -> float:
        return float(self.rng.uniform(0.01, 0.1))

    def conv(self, x: str, cin: int, cout: int, k: int, stride: int, group: int = 1,
             relu: bool = False) -> str:
        self.k += 1
        i = self.k
        icg = cin // group
        w = self.rng.standard_normal((cout, icg, k, k)) * 0.05
        s_w = np.abs(w).reshape(cout, -1).max(axis=1) / 127.0
        q_w = np.clip(np.rint(w / s_w[:, None, None, None]), -127, 127).astype(np.int8)
        s_x = self.scale[x]
        s_y = self.new_scale()
        bias = self.rng.standard_normal(cout) * 0.1
        q_b = np.rint(bias / (s_x * s_w)).astype(np.int32)
        mult = (s_x * s_w / s_y).astype(np.float32)
        b = self.b
        b.const(f"q{i}.w", q_w)
        b.const(f"q{i}.b", q_b)
        b.const(f"q{i}.m", mult)
        p = (k - 1) // 2
        attrs = dict(kernel_shape=[k, k], strides=[stride, stride], pads=[p] * 4, group=group,
                     dilations=[1, 1])
        if relu:
            attrs["activation"] = "Relu"
        y = b.node("QConv", [x, f"q{i}.w", f"q{i}.b", f"q{i}.m"], f"/q{i}/QConv_output_0",
                   name=f"/q{i}/QConv", **attrs)
        self.scale[y] = s_y
        return y

    def gelu(self, x: str) -> str:
        self.k += 1
        s_y = self.new_scale()
        t = self.b.const(f"gelu{self.k}.table", gelu_table(self.scale[x], s_y))
        y = self.b.node("QLut", [x, t], f"/gelu{self.k}/QLut_output_0", name=f"/gelu{self.k}/QLut")
        self.scale[y] = s_y
        return y

    def add(self, a: str, c: str) -> str:
        self.k += 1
        s_y = self.new_scale()
        y = self.b.node("QAdd", [a, c], f"/add{self.k}/QAdd_output_0", name=f"/add{self.k}/QAdd",
                        ma=float(np.float32(self.scale[a] / s_y)),
                        mb=float(np.float32(self.scale[c] / s_y)))
        self.scale[y] = s_y
        return y


def build_repvit_int8(*, batch: int = 32, seed: int = 0, num_classes: int = 1000,
                      widths=WIDTHS, depths=DEPTHS, image: int = 224) -> Graph:
    q = _QBuilder("repvit_int8", seed)
    b = q.b
    b.input("input", (batch, 3, image, image))
    s_in = q.new_scale()
    x = b.node("QuantizeLinear", ["input"], "/quant/QuantizeLinear_output_0", name="/quant",
               inv_scale=float(np.float32(1.0 / s_in)))
    q.scale[x] = s_in
    x = q.conv(x, 3, widths[0] // 2, 3, 2)
    x = q.gelu(x)
    x = q.conv(x, widths[0] // 2, widths[0], 3, 2)
    cin = widths[0]
    for si, (c, d) in enumerate(zip(widths, depths)):
        for bi in range(d):
            if bi == 0 and si > 0:
                x = q.conv(x, cin, cin, 3, 2, group=cin)          # token mixer, stride 2
                x = q.conv(x, cin, c, 1, 1)                       # to the new width
            else:
                x = q.conv(x, c, c, 3, 1, group=c)                # token mixer (re-parameterised)
            h = q.conv(x, c, 2 * c, 1, 1)                         # channel mixer
            h = q.gelu(h)
            h = q.conv(h, 2 * c, c, 1, 1)
            x = q.add(x, h)
            cin = c
    s_g = q.new_scale()
    hw = (image // 4 // 8) ** 2
    g = b.node("QGlobalAveragePool", [x], "/pool/QGlobalAveragePool_output_0", name="/pool",
               mult=float(np.float32(q.scale[x] / (hw * s_g))))
    q.scale[g] = s_g
    f = b.node("Flatten", [g], "/Flatten_output_0", name="/Flatten", axis=1)
    q.scale[f] = s_g
    w = q.rng.standard_normal((num_classes, cin)) * 0.05
    s_w = np.abs(w).max(axis=1) / 127.0
    q_w = np.clip(np.rint(w / s_w[:, None]), -127, 127).astype(np.int8)
    q_b = np.rint(q.rng.standard_normal(num_classes) * 0.1 / (s_g * s_w)).astype(np.int32)
    b.const("fc.w", q_w)
    b.const("fc.b", q_b)
    b.const("fc.m", (s_g * s_w).astype(np.float32))
    b.node("QGemm", [f, "fc.w", "fc.b", "fc.m"], "logits", name="/fc/QGemm", transB=1,
           out_dtype="float32")
    b.output("logits")
    return b.graph()


def make_input(batch: int = 32, seed: int = 0, image: int = 224) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((batch, 3, image, image)).astype(np.float32)


__all__ = ["build_repvit_int8", "make_input", "gelu_table", "DType"]
