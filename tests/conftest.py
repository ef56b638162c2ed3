"""Shared fixtures and markers.

``gpu`` tests need a visible HIP device and the built libmdlc_hip.so; they
are selected with ``-m gpu`` and skipped elsewhere. Everything else runs on
the CPU.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built shim")


def _hip_ok() -> bool:
    try:
        from mdlc_amd.codegen.hip.hiprtc_runtime import hip_available
        return hip_available()
    except Exception:
        return False


HIP_OK = _hip_ok()
requires_gpu = pytest.mark.skipif(not HIP_OK, reason="no HIP device visible")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


@pytest.fixture(scope="session")
def hip_ctx():
    if not HIP_OK:
        pytest.skip("no HIP device visible")
    from mdlc_amd.codegen.hip.hiprtc_runtime import HipContext
    return HipContext(0)


@pytest.fixture(params=["conv_bn_relu", "residual_block", "mlp"])
def model_case(request):
    name = request.param
    small = {"conv_bn_relu": dict(cin=3, cout=8, h=10, w=10),
             "residual_block": dict(c=4, h=8, w=8),
             "mlp": dict()}[name]
    return name, small


def build_graph(name, **kw):
    """(graph, feeds) for one of the reference's tiny models, feeds from the
    seed-0 dummy recipe."""
    from mdlc_amd.passes.shape_inference import make_dummy_feeds
    from mdlc_amd.tools import build_models as bm

    g = bm.build(name, **kw)
    return g, make_dummy_feeds(g, batch=1)
