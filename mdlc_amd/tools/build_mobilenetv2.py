"""MobileNetV2 (width 1.0) built straight into the IR (replaces the torchvision
export of mdlc/tools/build_mobilenetv2.py:14-35).

torchvision topology: a 3x3 stride-2 stem to 32 channels, 17 inverted
residual blocks with settings (t, c, n, s) = (1,16,1,1), (6,24,2,2),
(6,32,3,2), (6,64,4,2), (6,96,3,1), (6,160,3,2), (6,320,1,1), a 1x1 conv to
1280, global average pool, flatten and a 1280->1000 Gemm. ReLU6 is exported
as ``Clip`` whose bounds come from ``Constant`` nodes (the opset>=11 torch
pattern), so constant folding must resolve them before the Clip fuses.
Depthwise convs have ``group == channels``. Weight distributions and the
LSUV calibration are as in ``build_resnet18`` (the reference's MobileNetV2
exporter calibrates too, mdlc/tools/build_mobilenetv2.py:25-29).
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import Graph
from mdlc_amd.tools.graph_builder import GraphBuilder, bn_params, kaiming_normal

SETTINGS = [(1, 16, 1, 1), (6, 24, 2, 2), (6, 32, 3, 2), (6, 64, 4, 2),
            (6, 96, 3, 1), (6, 160, 3, 2), (6, 320, 1, 1)]


def build_mobilenetv2(*, batch: int = 1, seed: int = 0, num_classes: int = 1000,
                      calibrate: bool = True) -> Graph:
    b = GraphBuilder("mobilenetv2", seed)
    rng = b.rng
    b.input("input", (batch, 3, 224, 224))
    k = [0]

    def conv_bn(x, cin, cout, ksz, stride, group, relu6):
        k[0] += 1
        i = k[0]
        icg = cin // group
        w = b.const(f"conv{i}.weight", kaiming_normal(rng, (cout, icg, ksz, ksz), icg * ksz * ksz))
        p = (ksz - 1) // 2
        y = b.node("Conv", [x, w], f"/conv{i}/Conv_output_0", name=f"/conv{i}/Conv",
                   dilations=[1, 1], group=group, kernel_shape=[ksz, ksz], pads=[p] * 4,
                   strides=[stride, stride])
        prm = [b.const(f"bn{i}.{s}", a) for s, a in
               zip(("weight", "bias", "running_mean", "running_var"), bn_params(rng, cout))]
        y = b.node("BatchNormalization", [y] + prm, f"/bn{i}/BatchNormalization_output_0",
                   name=f"/bn{i}/BatchNormalization", epsilon=1e-5, momentum=0.9)
        if relu6:
            lo = b.node("Constant", [], f"/act{i}/Constant_output_0", name=f"/act{i}/Constant",
                        value=np.array(0.0, dtype=np.float32))
            hi = b.node("Constant", [], f"/act{i}/Constant_1_output_0", name=f"/act{i}/Constant_1",
                        value=np.array(6.0, dtype=np.float32))
            y = b.node("Clip", [y, lo, hi], f"/act{i}/Clip_output_0", name=f"/act{i}/Clip")
        return y

    x = conv_bn("input", 3, 32, 3, 2, 1, True)
    cin = 32
    blk = 0
    for t, c, n, s in SETTINGS:
        for j in range(n):
            stride = s if j == 0 else 1
            hidden = cin * t
            y = x
            if t != 1:
                y = conv_bn(y, cin, hidden, 1, 1, 1, True)
            y = conv_bn(y, hidden, hidden, 3, stride, hidden, True)
            y = conv_bn(y, hidden, c, 1, 1, 1, False)
            if stride == 1 and cin == c:
                y = b.node("Add", [x, y], f"/block{blk}/Add_output_0", name=f"/block{blk}/Add")
            x = y
            cin = c
            blk += 1
    x = conv_bn(x, cin, 1280, 1, 1, 1, True)
    x = b.node("GlobalAveragePool", [x], "/pool/GlobalAveragePool_output_0",
               name="/pool/GlobalAveragePool")
    x = b.node("Flatten", [x], "/Flatten_output_0", name="/Flatten", axis=1)
    bound = 1.0 / np.sqrt(1280.0)
    fw = b.const("classifier.weight", kaiming_normal(rng, (num_classes, 1280), 1280))
    fb = b.const("classifier.bias", rng.uniform(-bound, bound, num_classes).astype(np.float32))
    b.node("Gemm", [x, fw, fb], "logits", name="/classifier/Gemm", alpha=1.0, beta=1.0, transB=1)
    b.output("logits")
    g = b.graph()
    if calibrate:
        from mdlc_amd.tools.calibrate import lsuv_calibrate

        lsuv_calibrate(g, {"input": calibration_input(seed)})
    return g


def calibration_input(seed: int = 0) -> np.ndarray:
    """Two seeded N(0,1) images used only to calibrate the weights, so every
    batch size gets the same weights."""
    return np.random.default_rng(seed + 1000).standard_normal((2, 3, 224, 224)).astype(np.float32)


def make_input(batch: int = 1, seed: int = 0) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((batch, 3, 224, 224)).astype(np.float32)
