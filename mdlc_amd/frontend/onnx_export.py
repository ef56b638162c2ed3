"""IR ``Graph`` -> ONNX model bytes.

The reference exports its benchmark models from torch to ``.onnx`` files
(mdlc/tools/build_resnet18.py:14-30, build_mobilenetv2.py:14-35) and
compiles those. Here the models are built straight into the IR; this writer
turns such a graph (before optimization: only standard ONNX ops) into an
opset-17 ``.onnx`` file, so the same model can be fed to ``compile_onnx`` or
to any other ONNX consumer. Attribute types follow the Python values:
int -> INT, float -> FLOAT (float32 on the wire, as ONNX stores it),
str -> STRING, ndarray -> TENSOR, lists of those -> INTS/FLOATS/STRINGS.
"""

from __future__ import annotations

import os
from typing import Union

import numpy as np

from mdlc_amd.frontend import onnx_proto as P
from mdlc_amd.ir import DType, Graph

_CODES = {DType.FLOAT32: 1, DType.FLOAT16: 10, DType.INT64: 7, DType.INT32: 6, DType.INT8: 3,
          DType.BOOL: 9}


def _attribute(name: str, v) -> P.AttributeProto:
    a = P.AttributeProto(name=name)
    if isinstance(v, (bool, int, np.integer)):
        a.type, a.i = P.ATTR_INT, int(v)
    elif isinstance(v, (float, np.floating)):
        a.type, a.f = P.ATTR_FLOAT, float(v)
    elif isinstance(v, (str, bytes)):
        a.type, a.s = P.ATTR_STRING, v.encode("utf-8") if isinstance(v, str) else v
    elif isinstance(v, np.ndarray):
        a.type, a.t = P.ATTR_TENSOR, P.array_to_tensor("", v)
    elif isinstance(v, (list, tuple)) and all(isinstance(x, (str, bytes)) for x in v) and v:
        a.type = P.ATTR_STRINGS
        a.strings = [x.encode("utf-8") if isinstance(x, str) else x for x in v]
    elif isinstance(v, (list, tuple)) and all(isinstance(x, (bool, int, np.integer)) for x in v):
        a.type, a.ints = P.ATTR_INTS, [int(x) for x in v]
    elif isinstance(v, (list, tuple)) and all(isinstance(x, (int, float, np.number)) for x in v):
        a.type, a.floats = P.ATTR_FLOATS, [float(x) for x in v]
    else:
        raise TypeError(f"attribute {name!r}: a {type(v).__name__} has no ONNX attribute type")
    return a


def graph_to_model(graph: Graph, *, opset: int = 17) -> P.ModelProto:
    """A ModelProto of ``graph``: nodes in the graph's order, initializers as
    raw little-endian tensors, value_info for the graph inputs and outputs."""
    fused = [n.name for n in graph.nodes if n.is_fused]
    if fused:
        raise ValueError(f"fused nodes are not ONNX operators: {fused[:3]}; export the graph "
                         "before compile_graph optimizes it")

    def vinfo(name):
        info = graph.info(name)
        if info is None:
            return P.ValueInfoProto(name=name, elem_type=1)
        # a rank-0 TensorInfo in the IR is an edge whose shape is not known yet
        return P.ValueInfoProto(name=name, elem_type=_CODES[info.dtype], has_shape=info.rank > 0,
                                dims=[d if isinstance(d, str) else (None if d is None else int(d))
                                      for d in info.shape])

    g = P.GraphProto(name=graph.name)
    for n in graph.nodes:
        g.node.append(P.NodeProto(op_type=n.op_type, name=n.name, input=list(n.inputs),
                                  output=list(n.outputs),
                                  attribute=[_attribute(k, v) for k, v in n.attrs.items()]))
    g.initializer = [P.array_to_tensor(k, v) for k, v in graph.initializers.items()]
    g.input = [vinfo(e) for e in graph.inputs]
    g.output = [vinfo(e) for e in graph.outputs]
    return P.ModelProto(ir_version=8, producer_name="mdlc_amd", opset_import={"": opset}, graph=g)


def export_onnx(graph: Graph, path: Union[str, os.PathLike, None] = None, *,
                opset: int = 17) -> bytes:
    """Serialize ``graph`` as an ONNX model; write it to ``path`` if given."""
    data = P.serialize_model(graph_to_model(graph, opset=opset))
    if path is not None:
        with open(path, "wb") as f:
            f.write(data)
    return data
