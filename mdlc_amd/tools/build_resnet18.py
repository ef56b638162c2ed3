"""ResNet-18 built straight into the IR (replaces the torchvision ONNX export
of mdlc/tools/build_resnet18.py:14-30, which needs torchvision and onnx).

Node order and op types follow the torch export at opset 17 with constant
folding off: Conv (no bias) -> BatchNormalization -> Relu, MaxPool, residual
Add -> Relu, GlobalAveragePool, Flatten, Gemm(transB=1). The torch exporter
also emits 72 ``Identity`` nodes, one per BatchNorm parameter it
deduplicated; they are reproduced here (routing all but the first BN's
gamma/beta of each width through an Identity) so the imported graph has the
reference's 141 ops and constant folding has the same work to do.

Weights: conv and FC Kaiming-normal (fan-in), FC bias U(-1/sqrt(512),
1/sqrt(512)), BatchNorm gamma U(0.5,1.5), beta N(0,0.1), running_mean
N(0,0.1), running_var U(0.5,1.5); all from one seeded generator, and used
as drawn, like the reference's ResNet-18 exporter (mdlc/tools/
build_resnet18.py:14-30 applies no calibration). With these BatchNorm
statistics the residual stream grows to |x| of a few hundred by stage 4.
``calibrate=True`` instead rescales each Conv/Gemm to unit output std on a
fixed calibration input (the LSUV step mdlc/tools/export_utils.py:16-50
applies to the reference's MobileNetV2 and RepViT exports), which gives a
well-conditioned variant of the same network.
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import Graph
from mdlc_amd.tools.graph_builder import GraphBuilder, bn_params, kaiming_normal

STAGES = [(64, 1), (128, 2), (256, 2), (512, 2)]


def build_resnet18(*, batch: int = 1, seed: int = 0, num_classes: int = 1000,
                   identities: bool = True, calibrate: bool = False) -> Graph:
    b = GraphBuilder("resnet18", seed)
    rng = b.rng
    b.input("input", (batch, 3, 224, 224))
    first_bn_of_width: set = set()
    n_ident = [0]

    def conv(x, name, cin, cout, k, s, p):
        w = b.const(f"{name}.weight", kaiming_normal(rng, (cout, cin, k, k), cin * k * k))
        return b.node("Conv", [x, w], f"/{name}/Conv_output_0", name=f"/{name}/Conv",
                      dilations=[1, 1], group=1, kernel_shape=[k, k], pads=[p] * 4,
                      strides=[s, s])

    def bn(x, name, c):
        gamma, beta, mean, var = bn_params(rng, c)
        names = []
        for suffix, arr in (("weight", gamma), ("bias", beta), ("running_mean", mean),
                            ("running_var", var)):
            names.append(b.const(f"{name}.{suffix}", arr))
        if identities:
            direct = 2 if c not in first_bn_of_width else 0
            first_bn_of_width.add(c)
            for i in range(direct, 4):
                n_ident[0] += 1
                src = names[i]
                names[i] = b.node("Identity", [src], f"onnx::Identity_{n_ident[0]}",
                                  name=f"Identity_{n_ident[0]}")
        return b.node("BatchNormalization", [x] + names, f"/{name}/BatchNormalization_output_0",
                      name=f"/{name}/BatchNormalization", epsilon=1e-5, momentum=0.9)

    def relu(x, name):
        return b.node("Relu", [x], f"/{name}/Relu_output_0", name=f"/{name}/Relu")

    x = conv("input", "conv1", 3, 64, 7, 2, 3)
    x = bn(x, "bn1", 64)
    x = relu(x, "relu")
    x = b.node("MaxPool", [x], "/maxpool/MaxPool_output_0", name="/maxpool/MaxPool",
               ceil_mode=0, dilations=[1, 1], kernel_shape=[3, 3], pads=[1, 1, 1, 1],
               strides=[2, 2])
    cin = 64
    for si, (c, stride) in enumerate(STAGES, start=1):
        for bi in range(2):
            s = stride if bi == 0 else 1
            pre = f"layer{si}.{bi}"
            y = conv(x, f"{pre}.conv1", cin, c, 3, s, 1)
            y = bn(y, f"{pre}.bn1", c)
            y = relu(y, f"{pre}.relu")
            y = conv(y, f"{pre}.conv2", c, c, 3, 1, 1)
            y = bn(y, f"{pre}.bn2", c)
            if s != 1 or cin != c:
                sc = conv(x, f"{pre}.downsample.0", cin, c, 1, s, 0)
                sc = bn(sc, f"{pre}.downsample.1", c)
            else:
                sc = x
            y = b.node("Add", [y, sc], f"/{pre}/Add_output_0", name=f"/{pre}/Add")
            x = relu(y, f"{pre}.relu_1")
            cin = c
    x = b.node("GlobalAveragePool", [x], "/avgpool/GlobalAveragePool_output_0",
               name="/avgpool/GlobalAveragePool")
    x = b.node("Flatten", [x], "/Flatten_output_0", name="/Flatten", axis=1)
    bound = 1.0 / np.sqrt(512.0)
    fw = b.const("fc.weight", kaiming_normal(rng, (num_classes, 512), 512))
    fb = b.const("fc.bias", rng.uniform(-bound, bound, num_classes).astype(np.float32))
    b.node("Gemm", [x, fw, fb], "logits", name="/fc/Gemm", alpha=1.0, beta=1.0, transB=1)
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
    """The benchmark input: N(0,1) images, [batch, 3, 224, 224], float32."""
    return np.random.default_rng(seed).standard_normal((batch, 3, 224, 224)).astype(np.float32)
