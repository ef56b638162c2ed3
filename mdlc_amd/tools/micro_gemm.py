"""The fused GEMM+bias+ReLU micro-workloads: C = relu(A @ B + bias).

(M, N, K) are ResNet-18's im2col GEMM shapes at batch 1. A, B and bias are
drawn from N(0,1)/sqrt(K) with a fixed seed per shape. As a graph this is a
runtime input A [M,K], constant B [K,N] and bias [N], Gemm -> Relu, which the
passes fuse into one ``FusedGemmAct`` group.
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import Graph
from mdlc_amd.tools.graph_builder import GraphBuilder

SHAPES = [(1, 1000, 512), (3136, 64, 576), (784, 128, 1152), (196, 256, 2304), (49, 512, 4608)]


def shape_seed(M: int, N: int, K: int) -> int:
    return (M * 1_000_003 + N * 1009 + K) % (2**31)


def operands(M: int, N: int, K: int):
    rng = np.random.default_rng(shape_seed(M, N, K))
    s = 1.0 / np.sqrt(K)
    A = (rng.standard_normal((M, K)) * s).astype(np.float32)
    B = (rng.standard_normal((K, N)) * s).astype(np.float32)
    bias = (rng.standard_normal(N) * s).astype(np.float32)
    return A, B, bias


def build_micro_gemm(M: int, N: int, K: int) -> tuple:
    """(graph, feeds) for one micro shape."""
    A, B, bias = operands(M, N, K)
    b = GraphBuilder(f"gemm_{M}x{N}x{K}")
    b.input("A", (M, K))
    b.const("B", B)
    b.const("bias", bias)
    b.node("Gemm", ["A", "B", "bias"], "pre", name="gemm")
    b.node("Relu", ["pre"], "C", name="relu")
    b.output("C")
    return b.graph(), {"A": A}
