"""The C-ABI boundary and the code generator, without a GPU.

* libmdlc_hip.so loads and exports every entry point include/mdlc_hip.h
  declares; calls that need a device fail with an error code and a message
  instead of crashing (the reference's CudaError taxonomy,
  nvrtc_runtime.py:74-92).
* hipRTC compiles every generated module for gfx950 here (no device needed),
  and a broken source raises HipError carrying the compiler log
  (reference: NVRTC failure -> CudaError with the build log, :110-111).
* The packed launch-plan format round-trips through the C++ parser.
* Codegen emits what it claims: exact float literals, the reference's
  activation semantics, no host fallbacks.
"""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

from mdlc_amd.build import LIB_PATH, ROOT
from mdlc_amd.codegen.hip import hiprtc_runtime as R
from mdlc_amd.codegen.hip import templates as T
from mdlc_amd.compiler import compile_graph
from mdlc_amd.tools.build_mobilenetv2 import build_mobilenetv2
from mdlc_amd.tools.build_resnet18 import build_resnet18
from mdlc_amd.tools.micro_gemm import SHAPES, build_micro_gemm

HEADER = os.path.join(ROOT, "include", "mdlc_hip.h")


def declared_symbols() -> list:
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(mdlc_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB_PATH), "build with `python -m mdlc_amd.build`"
    lib = ctypes.CDLL(LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 25
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in mdlc_hip.h but not exported"
    assert set(syms) == set(R._SIGS), "ctypes bindings and header disagree"


def test_device_calls_fail_cleanly_without_device():
    if R.hip_available():
        pytest.skip("a device is visible")
    n = ctypes.c_int(-1)
    rc = R.lib().mdlc_device_count(ctypes.byref(n))
    assert n.value == 0 and (rc != 0 or n.value == 0)
    rc = R.lib().mdlc_sync()
    assert rc != 0 and b"mdlc_init" in R.lib().mdlc_last_error()
    with pytest.raises(R.HipError):
        R.HipContext(0)


def test_broken_source_raises_with_log():
    with pytest.raises(R.HipError) as ei:
        R.compile_code_object('extern "C" __global__ void k() { this is not hip; }', use_cache=False)
    assert "error" in str(ei.value).lower()


@pytest.mark.parametrize("mode", ["implicit", "im2col"])
@pytest.mark.parametrize("batch", [1, 32])
def test_resnet18_module_compiles_for_gfx950(mode, batch):
    c = compile_graph(build_resnet18(batch=batch, calibrate=False), batch=batch, conv_mode=mode)
    assert c.module.fallbacks() == []
    code = R.compile_code_object(c.module.sources())
    assert code[:4] == b"\x7fELF"
    for name in c.module.kernels:
        assert name.encode() in code


def test_mobilenetv2_and_micro_modules_compile():
    for fold in (True, False):
        c = compile_graph(build_mobilenetv2(batch=1, calibrate=False), fuse_residual=fold)
        kinds = {l.kind for l in c.module.plan}
        assert kinds >= {"conv", "dwconv", "gap"} and ("elementwise" in kinds) != fold
        R.compile_code_object(c.module.sources())
    for M, N, K in SHAPES:
        g, feeds = build_micro_gemm(M, N, K)
        R.compile_code_object(compile_graph(g, feeds=feeds).module.sources())


def test_plan_format_round_trips():
    recs = [(0x1000, (3, 1, 1), (256, 1, 1), 0, [R.Arg.ptr(0xdead0000), R.Arg.i32(-7),
                                                 R.Arg.i64(1 << 40), R.Arg.f32(0.5)]),
            (0x2000, (1, 2, 3), (64, 1, 1), 128, [])]
    p = R.Plan(recs)
    n = ctypes.c_int()
    assert R.lib().mdlc_plan_num_launches(p._h, ctypes.byref(n)) == 0 and n.value == 2
    p.close()
    bad = ctypes.create_string_buffer(b"XXXX" + b"\0" * 12)
    h = ctypes.c_void_p()
    assert R.lib().mdlc_plan_create(bad, 16, ctypes.byref(h)) != 0
    assert b"bad header" in R.lib().mdlc_last_error()
    blob = R.pack_plan(recs)[:-3]                   # truncated
    buf = ctypes.create_string_buffer(blob, len(blob))
    assert R.lib().mdlc_plan_create(buf, len(blob), ctypes.byref(h)) != 0


def test_exact_float_literals():
    for v in (0.1, 1 / 3, 6.0, -2.5e-8, 0.16666667):
        lit = T.flit(v)
        assert float.fromhex(lit[:-1]) == float(np.float32(v))


def test_activation_expressions_follow_numpy_semantics():
    assert T.activation_expr(None, "v", {}) == "v"
    assert T.activation_expr("Relu", "v", {}) == "fmaxf(v, 0.0f)"
    assert "/ 6.0f" in T.activation_expr("HardSwish", "v", {})          # x/6, not x*0.16666667
    assert ">=" in T.activation_expr("LeakyRelu", "v", {"alpha": 0.1})  # np.where(x >= 0, ...)
    clip = T.activation_expr("Clip", "v", {"clip_min": 0.0, "clip_max": None})
    assert "fmaxf" in clip and "fminf" not in clip
    with pytest.raises(NotImplementedError):
        T.activation_expr("Gelu", "v", {})


def test_unsupported_op_raises_instead_of_host_fallback():
    from mdlc_amd.tools.graph_builder import GraphBuilder

    b = GraphBuilder("shape")
    b.input("x", (2, 8))
    b.node("Shape", ["x"], "y")
    b.output("y")
    with pytest.raises(NotImplementedError, match="no device lowering"):
        compile_graph(b.graph())


def test_repvit_int8_module_compiles_and_is_channels_last():
    from mdlc_amd.tools.build_repvit_int8 import build_repvit_int8, make_input

    for fused, dw in ((True, "mfma"), (False, "vector")):
        c = compile_graph(build_repvit_int8(batch=2), feeds={"input": make_input(2)},
                          fuse_int8_epilogues=fused, int8_depthwise=dw)
        kinds = {l.kind for l in c.module.plan}
        assert kinds >= {"qgemm", "qgap"}
        assert ("quantize" in kinds) != fused and ("qconv_first" in kinds) == fused
        assert ("qlut" in kinds and "qadd" in kinds) != fused
        assert ("qdwconv" in kinds) == (dw == "vector")
        assert ("qmlp" in kinds) == fused                   # stages 1-3 fold at batch 2
        assert c.module.fallbacks() == []
        assert all(c.module.device_layout.get(l.outputs[0]) == "NHWC"
                   for l in c.module.plan if (l.kind in ("qdwconv", "qlut", "qadd", "qgemm")
                                              and l.meta.get("OH")) or l.kind in ("qmlp", "qconv_first"))
        R.compile_code_object(c.module.sources())


def test_code_object_cache_key_tracks_the_toolchain(monkeypatch):
    """Objects built by another hipRTC / HIP runtime are never reused: the
    toolchain versions are part of the cache key."""
    v = R.toolchain_version()
    assert v.startswith("hiprtc-") and "/hip-" in v
    src = 'extern "C" __global__ void k(float* p) { p[0] = 1.0f; }'
    k0 = R._cache_key(src, "a.hip", "gfx950", ("-O3",))
    monkeypatch.setattr(R, "_TOOLCHAIN", v + "-other")
    assert R._cache_key(src, "a.hip", "gfx950", ("-O3",)) != k0


@pytest.mark.gpu
def test_fresh_hiprtc_compile_on_the_device_runs(hip_ctx):
    """hipRTC on the device's own host (no cache): the micro GEMM module is
    compiled from source, loaded and run, and matches the oracle."""
    from gpu_util import assert_close
    from mdlc_amd.codegen.hip.hip_executor import HipExecutor
    from mdlc_amd.testing import DEVICE_TENSOR
    from oracle.reference import run_reference

    g, feeds = build_micro_gemm(*SHAPES[1])
    c = compile_graph(g, feeds=feeds)
    ex = HipExecutor(c.module, hip_ctx, use_cache=False)
    try:
        got = ex.run(feeds)["outputs"]
    finally:
        ex.close()
    want = run_reference(c.graph, feeds)
    for k in want:
        assert_close(k, got[k], want[k], DEVICE_TENSOR)
