"""The compile CLI (reference: mdlc/tools/compile.py:15-51) on the CPU:
report, emit, cost-model tuning, ONNX files in (and out, through the
exporter), and clear errors for missing or malformed files."""

from __future__ import annotations

import json

import pytest

from mdlc_amd.tools import compile as cli


def test_report_names_passes_kernels_and_planner(capsys):
    assert cli.main(["resnet18", "--report"]) == 0
    out = capsys.readouterr().out
    assert "compile report" in out and "HIP module" in out and "host fallbacks: none" in out
    assert "fused groups" in out


def test_emit_writes_the_hiprtc_translation_unit(tmp_path, capsys):
    path = tmp_path / "resnet18.hip"
    assert cli.main(["resnet18", "--emit", str(path)]) == 0
    src = path.read_text()
    assert 'extern "C" __global__' in src and "gemm_f32_mfma" in src
    assert "wrote generated HIP" in capsys.readouterr().out


def test_tune_without_a_device_uses_the_cost_model(tmp_path, capsys):
    cache = tmp_path / "sched.json"
    assert cli.main(["micro:196x256x2304", "--tune", "--cache", str(cache), "--budget", "4"]) == 0
    entries = json.loads(cache.read_text())
    assert list(entries) == ["196x256x2304"]
    assert "cost model" in capsys.readouterr().out or entries["196x256x2304"]["measured"]


def test_no_fold_keeps_the_reference_groups(capsys):
    assert cli.main(["resnet18", "--no-fold", "--report", "--conv-mode", "im2col"]) == 0
    out = capsys.readouterr().out
    assert "elementwisex8" in out and "im2colx20" in out


def test_onnx_file_compiles(capsys):
    from onnx_fixtures import fixture_path

    assert cli.main([fixture_path("resnet18_w4"), "--report"]) == 0
    out = capsys.readouterr().out
    assert "Graph 'main_graph': 69 nodes" in out and "host fallbacks: none" in out


def test_exported_model_compiles(tmp_path, capsys):
    from mdlc_amd.tools import export_onnx

    path = tmp_path / "micro.onnx"
    assert export_onnx.main(["micro:49x512x4608", "--out", str(path)]) == 0
    assert cli.main([str(path)]) == 0
    assert "gemm" in capsys.readouterr().out


def test_missing_or_malformed_onnx_fails_with_a_clear_message(tmp_path, capsys):
    assert cli.main(["model.onnx"]) == 2
    assert "model.onnx" in capsys.readouterr().err
    bad = tmp_path / "bad.onnx"
    bad.write_bytes(b"\x0a\x05ab")
    assert cli.main([str(bad)]) == 2
    assert "runs past the message" in capsys.readouterr().err


def test_unknown_model_name():
    with pytest.raises(SystemExit):
        cli.main(["vgg16"])


@pytest.mark.gpu
@pytest.mark.parametrize("model", ["micro:49x512x4608", "resnet18"])
def test_run_on_the_device_matches_the_oracle(model, tmp_path, capsys):
    """``--run`` compiles, runs on the device and writes the outputs, which
    match the oracle on the same feeds (network tier for the whole model)."""
    import numpy as np

    from mdlc_amd.compiler import compile_graph
    from mdlc_amd.testing import FP32_NETWORK, compare_arrays
    from oracle.reference import run_reference

    path = tmp_path / "out.npz"
    assert cli.main([model, "--run", "--save-outputs", str(path)]) == 0
    assert "ran on the device" in capsys.readouterr().out
    saved = np.load(path)
    feeds = {k[3:]: saved[k] for k in saved.files if k.startswith("in:")}
    graph, _ = cli.build_model(model, 1)
    want = run_reference(compile_graph(graph, feeds=feeds).graph, feeds)
    for name, ref in want.items():
        r = compare_arrays(name, saved[f"out:{name}"], ref, rtol=FP32_NETWORK.rtol, atol=FP32_NETWORK.atol)
        assert r.ok, str(r)
