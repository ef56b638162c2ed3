"""Write the ONNX fixtures of the frontend tests: small models exported by
torch's TorchScript ONNX exporter, with torch's own float32 outputs on a
seeded input as the expected values.

    python tests/golden/make_onnx_fixtures.py

The models have the reference's topologies (mdlc/tools/build_resnet18.py,
build_mobilenetv2.py exported torchvision's ResNet-18 and MobileNetV2;
mdlc/tools/build_models.py:19-116 hand-built conv_bn_relu, residual_block
and mlp), at reduced width so the files stay small; the exporter call is the
reference's (opset 17, do_constant_folding=False, named input/output).
torchvision is absent here, so the two networks are written out as torch
modules with torchvision's layer structure.

torch's exporter serializes the model in C++ and then hands the bytes to the
``onnx`` package only to splice in onnxscript custom functions; none of these
models has one, and ``onnx`` is not installed, so that step is replaced by the
identity for the duration of the export.

Each fixture is ``<name>.onnx`` plus ``<name>.npz`` with the feed(s) and
torch's outputs (``in:<name>``, ``out:<name>``).
"""

from __future__ import annotations

import io
import os

import numpy as np
import torch
from torch import nn

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "onnx")


class BasicBlock(nn.Module):
    def __init__(self, cin, cout, stride):
        super().__init__()
        self.conv1 = nn.Conv2d(cin, cout, 3, stride, 1, bias=False)
        self.bn1 = nn.BatchNorm2d(cout)
        self.relu = nn.ReLU(inplace=True)
        self.conv2 = nn.Conv2d(cout, cout, 3, 1, 1, bias=False)
        self.bn2 = nn.BatchNorm2d(cout)
        self.downsample = None
        if stride != 1 or cin != cout:
            self.downsample = nn.Sequential(nn.Conv2d(cin, cout, 1, stride, bias=False),
                                            nn.BatchNorm2d(cout))

    def forward(self, x):
        skip = x if self.downsample is None else self.downsample(x)
        y = self.relu(self.bn1(self.conv1(x)))
        return self.relu(self.bn2(self.conv2(y)) + skip)


class ResNet18(nn.Module):
    """torchvision.models.resnet18's layers, base width ``w``."""

    def __init__(self, w=64, num_classes=1000):
        super().__init__()
        self.conv1 = nn.Conv2d(3, w, 7, 2, 3, bias=False)
        self.bn1 = nn.BatchNorm2d(w)
        self.relu = nn.ReLU(inplace=True)
        self.maxpool = nn.MaxPool2d(3, 2, 1)
        cin, stages = w, []
        for i, c in enumerate((w, 2 * w, 4 * w, 8 * w)):
            stages.append(nn.Sequential(BasicBlock(cin, c, 1 if i == 0 else 2), BasicBlock(c, c, 1)))
            cin = c
        self.layer1, self.layer2, self.layer3, self.layer4 = stages
        self.avgpool = nn.AdaptiveAvgPool2d((1, 1))
        self.fc = nn.Linear(8 * w, num_classes)

    def forward(self, x):
        x = self.maxpool(self.relu(self.bn1(self.conv1(x))))
        x = self.layer4(self.layer3(self.layer2(self.layer1(x))))
        return self.fc(torch.flatten(self.avgpool(x), 1))


class InvertedResidual(nn.Module):
    def __init__(self, cin, cout, stride, t):
        super().__init__()
        hidden = cin * t
        layers = []
        if t != 1:
            layers += [nn.Conv2d(cin, hidden, 1, bias=False), nn.BatchNorm2d(hidden), nn.ReLU6(True)]
        layers += [nn.Conv2d(hidden, hidden, 3, stride, 1, groups=hidden, bias=False),
                   nn.BatchNorm2d(hidden), nn.ReLU6(True),
                   nn.Conv2d(hidden, cout, 1, bias=False), nn.BatchNorm2d(cout)]
        self.conv = nn.Sequential(*layers)
        self.use_res = stride == 1 and cin == cout

    def forward(self, x):
        return x + self.conv(x) if self.use_res else self.conv(x)


class MobileNetV2(nn.Module):
    """torchvision.models.mobilenet_v2's layers (inverted residual settings
    t, c, n, s; channels rounded to multiples of 8), width ``mult``, with a
    narrower last conv so the file stays small."""

    SETTINGS = [(1, 16, 1, 1), (6, 24, 2, 2), (6, 32, 3, 2), (6, 64, 4, 2), (6, 96, 3, 1),
                (6, 160, 3, 2), (6, 320, 1, 1)]

    def __init__(self, mult=0.125, last=128, num_classes=10):
        super().__init__()

        def r8(v):
            n = max(8, int(v + 4) // 8 * 8)
            return n + 8 if n < 0.9 * v else n

        cin = r8(32 * mult)
        feats = [nn.Sequential(nn.Conv2d(3, cin, 3, 2, 1, bias=False), nn.BatchNorm2d(cin),
                               nn.ReLU6(True))]
        for t, c, n, s in self.SETTINGS:
            for i in range(n):
                feats.append(InvertedResidual(cin, r8(c * mult), s if i == 0 else 1, t))
                cin = r8(c * mult)
        feats.append(nn.Sequential(nn.Conv2d(cin, last, 1, bias=False), nn.BatchNorm2d(last),
                                   nn.ReLU6(True)))
        self.features = nn.Sequential(*feats)
        self.classifier = nn.Sequential(nn.Dropout(0.2), nn.Linear(last, num_classes))

    def forward(self, x):
        x = nn.functional.adaptive_avg_pool2d(self.features(x), (1, 1))
        return self.classifier(torch.flatten(x, 1))


class ConvBnRelu(nn.Module):
    def __init__(self, cin=3, cout=8, k=3):
        super().__init__()
        self.conv = nn.Conv2d(cin, cout, k, 1, k // 2)
        self.bn = nn.BatchNorm2d(cout)

    def forward(self, x):
        return torch.relu(self.bn(self.conv(x)))


class ResidualBlock(nn.Module):
    def __init__(self, c=8):
        super().__init__()
        self.a, self.a_bn = nn.Conv2d(c, c, 3, 1, 1, bias=False), nn.BatchNorm2d(c)
        self.b, self.b_bn = nn.Conv2d(c, c, 3, 1, 1, bias=False), nn.BatchNorm2d(c)

    def forward(self, x):
        y = torch.relu(self.a_bn(self.a(x)))
        return torch.relu(self.b_bn(self.b(y)) + x)


class Mlp(nn.Module):
    def __init__(self, din=16, dh=32, dout=8):
        super().__init__()
        self.fc1, self.fc2 = nn.Linear(din, dh), nn.Linear(dh, dout)

    def forward(self, x):
        return self.fc2(torch.relu(self.fc1(x)))


def randomize(model, seed):
    """BatchNorm statistics in the benchmark distributions (gamma U(0.5,1.5),
    beta/mean N(0,0.1), var U(0.5,1.5)) and He-normal conv/linear weights,
    so that every folded constant matters and activations stay O(1)."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, nn.BatchNorm2d):
                c = m.num_features
                m.weight.copy_(torch.rand(c, generator=g) + 0.5)
                m.bias.copy_(torch.randn(c, generator=g) * 0.1)
                m.running_mean.copy_(torch.randn(c, generator=g) * 0.1)
                m.running_var.copy_(torch.rand(c, generator=g) + 0.5)
            elif isinstance(m, (nn.Conv2d, nn.Linear)):
                fan_in = m.weight[0].numel()
                m.weight.copy_(torch.randn(m.weight.shape, generator=g) * (2.0 / fan_in) ** 0.5)
                if m.bias is not None:
                    m.bias.copy_(torch.randn(m.bias.shape, generator=g) * 0.1)
    return model


def export(name, model, x, *, in_name="input", out_name="logits", dynamic_batch=False):
    from torch.onnx._internal.torchscript_exporter import onnx_proto_utils

    model.eval()
    buf = io.BytesIO()
    splice = onnx_proto_utils._add_onnxscript_fn
    onnx_proto_utils._add_onnxscript_fn = lambda model_bytes, custom_opsets: model_bytes
    try:
        torch.onnx.export(model, torch.from_numpy(x), buf, input_names=[in_name],
                          output_names=[out_name], opset_version=17, do_constant_folding=False,
                          dynamic_axes=({in_name: {0: "batch"}, out_name: {0: "batch"}}
                                        if dynamic_batch else None), dynamo=False)
    finally:
        onnx_proto_utils._add_onnxscript_fn = splice
    with open(os.path.join(HERE, name + ".onnx"), "wb") as f:
        f.write(buf.getvalue())
    feeds = {in_name: x}
    if dynamic_batch:                     # a second batch size for the symbolic dim
        feeds = {in_name: x, in_name + "@3": np.concatenate([x, x[:1] * 0.5, -x[:1]])}
    outs = {}
    with torch.no_grad():
        for k, v in feeds.items():
            outs["out:" + out_name + k[len(in_name):]] = model(torch.from_numpy(v)).numpy()
    np.savez(os.path.join(HERE, name + ".npz"), **{"in:" + k: v for k, v in feeds.items()}, **outs)
    print(f"{name}: {len(buf.getvalue())} bytes")


def main():
    os.makedirs(HERE, exist_ok=True)
    torch.manual_seed(0)
    rng = np.random.default_rng(0)

    def img(*shape):
        return rng.standard_normal(shape).astype(np.float32)

    # torchvision's initial BatchNorm state (weight 1, bias 0, mean 0, var 1):
    # the exporter shares equal initializers through Identity nodes, as in
    # the reference's exported ResNet-18
    export("resnet18_w4_init", ResNet18(4, 10), img(1, 3, 64, 64))
    export("resnet18_w4", randomize(ResNet18(4, 10), 1), img(2, 3, 64, 64))
    export("mobilenetv2_x0125",randomize(MobileNetV2(), 2), img(1, 3, 64, 64))
    export("conv_bn_relu", randomize(ConvBnRelu(), 3), img(1, 3, 16, 16), in_name="x",
           out_name="y")
    export("residual_block", randomize(ResidualBlock(), 4), img(1, 8, 16, 16), in_name="x",
           out_name="y")
    export("mlp", randomize(Mlp(), 5), img(4, 16), in_name="x", out_name="y", dynamic_batch=True)


if __name__ == "__main__":
    main()
