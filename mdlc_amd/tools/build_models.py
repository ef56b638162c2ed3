"""The reference's three tiny test models, built straight into the IR.

Same topologies, shapes, seeds and weight distributions as
mdlc/tools/build_models.py:19-116 (conv_bn_relu, residual_block, mlp); the
random draws follow the same per-model generator sequence.
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import Graph
from mdlc_amd.tools.graph_builder import GraphBuilder


def conv_bn_relu_model(*, n=1, cin=3, cout=8, h=16, w=16, k=3, seed=0) -> Graph:
    """Conv -> BatchNormalization -> Relu (build_models.py:19-52)."""
    b = GraphBuilder("conv_bn_relu")
    rng = np.random.default_rng(seed)
    pad = k // 2
    weight = rng.standard_normal((cout, cin, k, k)).astype(np.float32) * 0.1
    bias = rng.standard_normal(cout).astype(np.float32) * 0.1
    gamma = rng.standard_normal(cout).astype(np.float32) * 0.2 + 1.0
    beta = rng.standard_normal(cout).astype(np.float32) * 0.1
    mean = rng.standard_normal(cout).astype(np.float32) * 0.1
    var = np.abs(rng.standard_normal(cout).astype(np.float32)) + 0.5
    for nm, arr in (("w", weight), ("b", bias), ("gamma", gamma), ("beta", beta),
                    ("mean", mean), ("var", var)):
        b.const(nm, arr)
    b.input("x", (n, cin, h, w))
    b.node("Conv", ["x", "w", "b"], "conv_out", name="conv",
           kernel_shape=[k, k], pads=[pad] * 4, strides=[1, 1])
    b.node("BatchNormalization", ["conv_out", "gamma", "beta", "mean", "var"], "bn_out",
           name="bn", epsilon=1e-5)
    b.node("Relu", ["bn_out"], "y", name="relu")
    b.output("y")
    return b.graph()


def residual_block_model(*, n=1, c=8, h=16, w=16, seed=1) -> Graph:
    """Two conv+BN paths joined by a residual Add -> Relu (build_models.py:55-93)."""
    bld = GraphBuilder("residual_block")
    rng = np.random.default_rng(seed)
    for tag in ("a", "b"):
        bld.const(f"w_{tag}", rng.standard_normal((c, c, 3, 3)).astype(np.float32) * 0.1)
        bld.const(f"gamma_{tag}", rng.standard_normal(c).astype(np.float32) * 0.2 + 1.0)
        bld.const(f"beta_{tag}", rng.standard_normal(c).astype(np.float32) * 0.1)
        bld.const(f"mean_{tag}", rng.standard_normal(c).astype(np.float32) * 0.1)
        bld.const(f"var_{tag}", np.abs(rng.standard_normal(c).astype(np.float32)) + 0.5)
    bld.input("x", (n, c, h, w))
    for tag, src in (("a", "x"), ("b", "a_relu")):
        bld.node("Conv", [src, f"w_{tag}", ""], f"{tag}_conv", name=f"conv_{tag}",
                 kernel_shape=[3, 3], pads=[1, 1, 1, 1])
        bld.node("BatchNormalization", [f"{tag}_conv", f"gamma_{tag}", f"beta_{tag}",
                                        f"mean_{tag}", f"var_{tag}"], f"{tag}_bn", name=f"bn_{tag}")
        if tag == "a":
            bld.node("Relu", ["a_bn"], "a_relu", name="relu_a")
    bld.node("Add", ["b_bn", "x"], "sum", name="add")
    bld.node("Relu", ["sum"], "y", name="relu_out")
    bld.output("y")
    return bld.graph()


def mlp_model(*, n=4, din=16, dh=32, dout=8, seed=2) -> Graph:
    """Gemm(transB) -> Relu -> Gemm(transB) (build_models.py:96-116)."""
    b = GraphBuilder("mlp")
    rng = np.random.default_rng(seed)
    b.const("w1", rng.standard_normal((dh, din)).astype(np.float32) * 0.1)
    b.const("b1", rng.standard_normal(dh).astype(np.float32) * 0.1)
    b.const("w2", rng.standard_normal((dout, dh)).astype(np.float32) * 0.1)
    b.const("b2", rng.standard_normal(dout).astype(np.float32) * 0.1)
    b.input("x", (n, din))
    b.node("Gemm", ["x", "w1", "b1"], "h1", name="fc1", transB=1)
    b.node("Relu", ["h1"], "h1r", name="relu1")
    b.node("Gemm", ["h1r", "w2", "b2"], "y", name="fc2", transB=1)
    b.output("y")
    return b.graph()


_REGISTRY = {
    "conv_bn_relu": conv_bn_relu_model,
    "residual_block": residual_block_model,
    "mlp": mlp_model,
}


def build(name: str, **kw) -> Graph:
    return _REGISTRY[name](**kw)
