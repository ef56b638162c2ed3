"""The torch-exported ONNX fixtures under tests/golden/onnx (written by
tests/golden/make_onnx_fixtures.py): paths and the feeds/outputs torch
computed for them."""

from __future__ import annotations

import os

import numpy as np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "onnx")
NAMES = ["conv_bn_relu", "residual_block", "mlp", "resnet18_w4", "resnet18_w4_init",
         "mobilenetv2_x0125"]


def fixture_path(name: str) -> str:
    return os.path.join(HERE, name + ".onnx")


def fixture_cases(name: str):
    """[(feeds, expected outputs)], one per feed set of the fixture (the
    dynamic-batch model has two batch sizes)."""
    z = np.load(os.path.join(HERE, name + ".npz"))
    cases = {}
    for k in z.files:
        kind, key = k.split(":", 1)
        base, _, tag = key.partition("@")
        feeds, outs = cases.setdefault(tag, ({}, {}))
        (feeds if kind == "in" else outs)[base] = z[k]
    return [cases[t] for t in sorted(cases)]
