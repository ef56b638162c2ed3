"""Graph IR consumed by the passes, the planner and the HIP codegen."""

from mdlc_amd.ir.tensor import DType, TensorInfo
from mdlc_amd.ir.node import Node
from mdlc_amd.ir.graph import Graph
from mdlc_amd.ir.verify import GraphVerifyError, verify_graph

__all__ = ["DType", "TensorInfo", "Node", "Graph", "GraphVerifyError", "verify_graph"]
