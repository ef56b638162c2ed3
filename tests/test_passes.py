"""Graph passes: numerics preserved, fusion structure, legality, and the
reference's published known answers for ResNet-18.

Mirrors tests/test_passes.py:27-185 of the reference (on IR-direct models,
since `onnx` is not part of this stack) plus the structural KATs of
docs/GAPS.md:17-19: 141 -> 32 ops, 17 fused groups (9 FusedConvAct + 8
FusedElementwise), and the planner's 13.119 -> 4.594 MiB in 3 buffers.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import build_graph
from mdlc_amd.compiler import compile_graph
from mdlc_amd.ir import verify_graph
from mdlc_amd.passes import (
    ConstantFolding, DeadCodeElimination, FuseActivation, FuseConvBN, FuseElementwise, default_pipeline,
)
from mdlc_amd.passes.shape_inference import infer_shapes
from mdlc_amd.runtime import plan_memory
from mdlc_amd.testing import BITWISE, FP32_NETWORK, FP32_SAME_ORDER, compare_arrays
from mdlc_amd.tools.build_mobilenetv2 import build_mobilenetv2
from mdlc_amd.tools.build_resnet18 import build_resnet18
from mdlc_amd.tools.graph_builder import GraphBuilder
from oracle.reference import run_reference


def make_pass_verifier(feeds, golden, tol=FP32_NETWORK):
    """The reference's per-pass verifier (testing/harness.py:127-149), built
    from the oracle on the test side and injected into the pipeline."""
    def verify(graph, name):
        verify_graph(graph, context=name)
        got = run_reference(graph, feeds)
        for o in graph.outputs:
            r = compare_arrays(o, got[o], golden[o], rtol=tol.rtol, atol=tol.atol)
            assert r.ok or "VACUOUS" in r.detail, f"pass {name!r} broke numerics: {r}"
    return verify


def test_pipeline_preserves_numerics(model_case):
    name, kw = model_case
    g, feeds = build_graph(name, **kw)
    golden = run_reference(g.clone(), feeds)
    g2 = default_pipeline(verify=make_pass_verifier(feeds, golden)).run(g)
    out = run_reference(g2, feeds)
    for o in g2.outputs:
        np.testing.assert_allclose(out[o], golden[o], rtol=FP32_NETWORK.rtol, atol=FP32_NETWORK.atol)


def test_conv_bn_relu_fuses_to_single_node():
    g, _ = build_graph("conv_bn_relu")
    g = default_pipeline().run(g)
    assert [n.op_type for n in g.nodes] == ["FusedConvAct"]
    assert g.nodes[0].attrs["activation"] == "Relu"


def test_conv_bn_fold_is_arithmetic_only():
    g, feeds = build_graph("conv_bn_relu")
    before = run_reference(g.clone(), feeds)
    assert FuseConvBN().run(g)
    assert not any(n.op_type == "BatchNormalization" for n in g.nodes)
    after = run_reference(g, feeds)
    for o in g.outputs:
        np.testing.assert_allclose(after[o], before[o], rtol=FP32_SAME_ORDER.rtol,
                                   atol=FP32_SAME_ORDER.atol)


def test_bn_fold_constants_are_bitwise_the_reference_formula():
    """w' = w * (g / sqrt(v + eps)) and b' = b*s + (beta - m*s), float32 ops in
    that order (fuse_conv_bn.py:53-68), checked against float64-free NumPy."""
    g, _ = build_graph("conv_bn_relu")
    init = dict(g.initializers)
    FuseConvBN().run(g)
    s = init["gamma"] / np.sqrt(init["var"] + 1e-5)
    np.testing.assert_array_equal(g.initializers["w_bnfold"], init["w"] * s.reshape(-1, 1, 1, 1))
    np.testing.assert_array_equal(g.initializers["conv_bias_bnfold"],
                                  init["b"] * s + (init["beta"] - init["mean"] * s))


def test_elementwise_fusion_groups_add_relu():
    g, _ = build_graph("residual_block", c=4, h=8, w=8)
    g = default_pipeline().run(g)
    fe = [n for n in g.nodes if n.op_type == "FusedElementwise"]
    assert len(fe) == 1
    assert [n.op_type for n in fe[0].attrs["subgraph"]] == ["Add", "Relu"]


def test_fusion_respects_multiple_consumers():
    g, _ = build_graph("residual_block", c=4, h=8, w=8)
    assert g.use_count()["x"] >= 2
    g2 = default_pipeline().run(g)
    assert len(g2.consumers()["x"]) >= 2


def test_constant_folding_removes_const_subgraph():
    b = GraphBuilder("constfold")
    b.const("a", np.full(4, 2.0, np.float32))
    b.const("b", np.full(4, 3.0, np.float32))
    b.input("x", (4,))
    b.node("Add", ["a", "b"], "c")
    b.node("Mul", ["x", "c"], "y")
    b.output("y")
    g = b.graph()
    assert ConstantFolding().run(g)
    assert not any(n.op_type == "Add" for n in g.nodes)
    assert g.is_constant("c")
    out = run_reference(g, {"x": np.ones(4, np.float32)})
    np.testing.assert_allclose(out["y"], np.full(4, 5.0), rtol=BITWISE.rtol, atol=BITWISE.atol)


def _clip_from_constants_model():
    """Conv -> Clip(0,6) with bounds from Constant nodes (the opset>=11 export
    pattern that once fused into an identity in the reference)."""
    rng = np.random.default_rng(7)
    b = GraphBuilder("clip_const")
    b.input("x", (1, 3, 8, 8))
    b.const("w", rng.standard_normal((4, 3, 3, 3)).astype(np.float32))
    b.node("Constant", [], "lo", value=np.array(0.0, np.float32))
    b.node("Constant", [], "hi", value=np.array(6.0, np.float32))
    b.node("Conv", ["x", "w"], "c", kernel_shape=[3, 3], pads=[1, 1, 1, 1])
    b.node("Clip", ["c", "lo", "hi"], "y")
    b.output("y")
    return b.graph()


def test_clip_with_unresolvable_bounds_is_not_fused():
    g = _clip_from_constants_model()
    FuseActivation().run(g)
    assert any(n.op_type == "Clip" for n in g.nodes)


def test_clip_bounds_resolved_through_pipeline():
    g = _clip_from_constants_model()
    feeds = {"x": np.random.default_rng(8).standard_normal((1, 3, 8, 8)).astype(np.float32) * 3}
    golden = run_reference(g.clone(), feeds)
    g = default_pipeline(verify=make_pass_verifier(feeds, golden)).run(g)
    fused = [n for n in g.nodes if n.op_type == "FusedConvAct"]
    assert len(fused) == 1
    assert fused[0].attrs["clip_min"] == 0.0 and fused[0].attrs["clip_max"] == 6.0
    out = run_reference(g, feeds)["y"]
    assert out.min() >= 0.0 and out.max() <= 6.0
    np.testing.assert_allclose(out, golden["y"], rtol=FP32_SAME_ORDER.rtol, atol=FP32_SAME_ORDER.atol)


def test_dce_drops_dead_nodes():
    b = GraphBuilder("dce")
    b.input("x", (4,))
    b.node("Relu", ["x"], "live")
    b.node("Sigmoid", ["x"], "dead")
    b.output("live")
    g = b.graph()
    DeadCodeElimination().run(g)
    assert [n.op_type for n in g.nodes] == ["Relu"]


# ----- the reference's published structural numbers ---------------------------

@pytest.fixture(scope="module")
def resnet18_b1():
    g = build_resnet18(batch=1, calibrate=False)
    n0 = len(g.nodes)
    hist0 = g.op_histogram()
    g = default_pipeline().run(g)
    infer_shapes(g)
    return n0, hist0, g


def test_resnet18_op_counts_match_reference(resnet18_b1):
    n0, hist0, g = resnet18_b1
    assert n0 == 141 and hist0["Identity"] == 72 and hist0["BatchNormalization"] == 20
    assert len(g.nodes) == 32
    hist = g.op_histogram()
    assert hist["FusedConvAct"] == 9 and hist["FusedElementwise"] == 8
    assert sum(1 for n in g.nodes if n.is_fused) == 17


def test_resnet18_planner_matches_reference(resnet18_b1):
    _, _, g = resnet18_b1
    p = plan_memory(g)
    mib = 1024 * 1024
    assert len(p.buffers) == 3
    assert round(p.naive_activation_bytes / mib, 3) == 13.119
    assert round(p.planned_activation_bytes / mib, 3) == 4.594
    assert p.planned_activation_bytes < 0.6 * p.naive_activation_bytes


def test_resnet18_planner_at_batch32():
    g = default_pipeline().run(build_resnet18(batch=32, calibrate=False))
    infer_shapes(g)
    p = plan_memory(g)
    assert round(p.naive_activation_bytes / 2**20, 3) == 419.810
    assert round(p.planned_activation_bytes / 2**20, 3) == 147.000


def test_resnet18_explicit_lowering_has_reference_launch_count():
    """12 distinct kernels / 52 launches in the reference (docs/GAPS.md:18);
    the same 52 launches here with the reference's pass pipeline alone, none
    of them on the host — and 43 once the backend folds the 8 residual
    Add+Relu groups into the conv epilogues and lets the pool write the
    flattened classifier input."""
    sched = __import__("mdlc_amd.codegen.schedule", fromlist=["x"]).MfmaSchedule(64, 64, 16, 2, 2, 32)
    c = compile_graph(build_resnet18(batch=1, calibrate=False), conv_mode="im2col",
                      schedule_fn=lambda n, mnk: sched, fuse_residual=False)
    kinds = [l.kind for l in c.module.plan]
    assert len(kinds) == 52
    assert kinds.count("im2col") == 20 and kinds.count("gemm") == 21
    assert kinds.count("elementwise") == 8
    assert c.module.fallbacks() == []
    c = compile_graph(build_resnet18(batch=1, calibrate=False), conv_mode="im2col",
                      schedule_fn=lambda n, mnk: sched)
    kinds = [l.kind for l in c.module.plan]
    assert len(kinds) == 43 and kinds.count("elementwise") == 0 and "copy" not in kinds


def test_mobilenetv2_structure():
    g = build_mobilenetv2(batch=1, calibrate=False)
    hist = g.op_histogram()
    assert hist["Conv"] == 52 and hist["Clip"] == 35 and hist["Add"] == 10
    assert sum(1 for n in g.nodes if n.op_type == "Conv" and n.attrs["group"] > 1) == 17
    g = default_pipeline().run(g)
    hist = g.op_histogram()
    assert hist.get("Clip", 0) == 0 and hist.get("Constant", 0) == 0
    assert hist["FusedConvAct"] == 35


def test_shape_rules_agree_with_oracle_shapes():
    g = default_pipeline().run(build_mobilenetv2(batch=2, calibrate=False))
    x = np.random.default_rng(0).standard_normal((2, 3, 224, 224)).astype(np.float32)
    infer_shapes(g, {"input": x})
    env = run_reference(g, {"input": x}, return_all=True)
    for k, v in env.items():
        assert tuple(g.info(k).shape) == v.shape, k
        assert g.info(k).dtype == str(v.dtype), k
