"""ONNX files compiled and run on the device: the torch-exported fixtures
(tests/golden/onnx) through ``compile_onnx`` and the executor. Every fused
group's tensor is held to the oracle at rtol 1e-4 / atol 1e-5, and the
outputs to torch's own float32 outputs at the network tier (the
reference's end-to-end check against onnxruntime,
tests/test_frontend_reference.py:29-41, with torch as the independent
implementation)."""

from __future__ import annotations

import pytest

from gpu_util import assert_close
from mdlc_amd.codegen.hip.hip_executor import HipExecutor
from mdlc_amd.compiler import compile_onnx
from mdlc_amd.testing import DEVICE_TENSOR, FP32_NETWORK
from onnx_fixtures import NAMES, fixture_cases, fixture_path
from oracle.reference import run_reference

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", NAMES)
def test_onnx_fixture_on_the_device(name, hip_ctx):
    for feeds, torch_out in fixture_cases(name):
        c = compile_onnx(fixture_path(name), feeds=feeds)
        assert c.module.fallbacks() == []
        want = run_reference(c.graph, feeds, return_all=True)
        ex = HipExecutor(c.module, hip_ctx)
        try:
            ex._upload_feeds(feeds)
            got = ex.run_isolated(want)
            outs = ex.run(feeds)["outputs"]
        finally:
            ex.close()
        for t, v in got.items():
            assert_close(t, v, want[t], DEVICE_TENSOR)
        for k, v in torch_out.items():
            assert_close(k, outs[k], v, FP32_NETWORK)
