"""Two independent implicit-GEMM convolutions in one launch, on the device:
the paired launch computes every tile with the same code as the two
launches, so its outputs equal theirs bit for bit, and both meet the oracle
(a synthetic pair of convs on one input, and ResNet-18 at batch 32, whose
stage-2 stride-2 conv and downsample are paired)."""

from __future__ import annotations

import numpy as np
import pytest

from gpu_util import assert_close, device_run
from test_conv_pair import TILED, _Tiled, _two_convs
from mdlc_amd.tools.build_resnet18 import build_resnet18, make_input

pytestmark = pytest.mark.gpu


def test_paired_convs_equal_the_two_launches(hip_ctx):
    g, feeds = _two_convs()
    c, got, want = device_run(g, feeds, ctx=hip_ctx, schedule_fn=_Tiled(TILED), winograd=False)
    assert [l.kind for l in c.module.plan] == ["conv_pair"]
    g2, _ = _two_convs()
    c2, got2, _ = device_run(g2, feeds, ctx=hip_ctx, schedule_fn=_Tiled(TILED), winograd=False,
                             pair_convs=False)
    assert [l.kind for l in c2.module.plan] == ["conv", "conv"]
    for name in ("y1", "y2"):
        np.testing.assert_array_equal(got[name], got2[name], err_msg=name)
        assert_close(name, got[name], want[name])


def test_resnet18_b32_paired_equals_unpaired(hip_ctx):
    feeds = {"input": make_input(32)}
    c, got, want = device_run(build_resnet18(batch=32, calibrate=True), feeds, ctx=hip_ctx,
                              all_tensors=True)
    assert sum(l.kind == "conv_pair" for l in c.module.plan) == 1
    c2, got2, _ = device_run(build_resnet18(batch=32, calibrate=True), feeds, ctx=hip_ctx,
                             all_tensors=True, pair_convs=False)
    assert "conv_pair" not in {l.kind for l in c2.module.plan}
    names = [k for k in got if k in got2 and k not in c.graph.initializers]
    assert "logits" in names and "/layer2.0.downsample.1/BatchNormalization_output_0" in names
    for k in names:
        np.testing.assert_array_equal(got[k], got2[k], err_msg=k)
    p = next(l for l in c.module.plan if l.kind == "conv_pair")
    for k in p.outputs:
        assert_close(k, got[k], want[k])
