"""A small helper for building IR graphs directly (no ONNX needed).

The reference builds its models with ``onnx.helper`` and imports them
(mdlc/tools/build_models.py, mdlc/frontend/onnx_importer.py). ``onnx`` is not
part of this stack, so models are written straight into the IR with the same
op types, attribute names and edge conventions an ONNX import produces.
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import DType, Graph, Node, TensorInfo


class GraphBuilder:
    def __init__(self, name: str, seed: int = 0) -> None:
        self.g = Graph(name)
        self.rng = np.random.default_rng(seed)
        self._n = 0

    def input(self, name: str, shape, dtype: str = DType.FLOAT32) -> str:
        self.g.inputs.append(name)
        self.g.set_info(TensorInfo(name, dtype, tuple(shape)))
        return name

    def output(self, name: str) -> None:
        self.g.outputs.append(name)

    def const(self, name: str, array) -> str:
        self.g.set_initializer(name, np.asarray(array))
        return name

    def node(self, op: str, inputs, outputs=None, name: str = "", **attrs) -> str:
        self._n += 1
        if outputs is None:
            outputs = [f"{name or op.lower()}_{self._n}_out"]
        elif isinstance(outputs, str):
            outputs = [outputs]
        self.g.add_node(Node(op, list(inputs), list(outputs), dict(attrs), name or f"{op}_{self._n}"))
        return outputs[0]

    def graph(self) -> Graph:
        return self.g


def kaiming_normal(rng, shape, fan_in: int) -> np.ndarray:
    """N(0, 2/fan_in): He initialisation for ReLU networks."""
    return (rng.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(np.float32)


def bn_params(rng, c: int):
    """BatchNorm parameters with the distributions the benchmark configs name:
    gamma U(0.5,1.5), beta N(0,0.1), running_mean N(0,0.1), running_var U(0.5,1.5)."""
    gamma = rng.uniform(0.5, 1.5, c).astype(np.float32)
    beta = (rng.standard_normal(c) * 0.1).astype(np.float32)
    mean = (rng.standard_normal(c) * 0.1).astype(np.float32)
    var = rng.uniform(0.5, 1.5, c).astype(np.float32)
    return gamma, beta, mean, var
