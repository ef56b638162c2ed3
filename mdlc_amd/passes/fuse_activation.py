"""Fuse a pointwise activation into the Conv/Gemm that produces its input.

Conv -> act becomes ``FusedConvAct`` and Gemm -> act becomes ``FusedGemmAct``
(mdlc/passes/fuse_activation.py:17-94). The activation runs in the GEMM
epilogue, so its parameters must be compile-time constants: a Clip whose
bound is a runtime tensor is left unfused rather than silently dropped.
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import Graph, Node
from mdlc_amd.passes.base import Pass

ACTIVATIONS = {"Relu", "Clip", "Sigmoid", "Tanh", "HardSwish", "HardSigmoid", "LeakyRelu"}
_FUSED_NAME = {"Conv": "FusedConvAct", "Gemm": "FusedGemmAct"}


def _const_scalar(graph: Graph, node: Node, slot: int, fallback):
    """(ok, value) for an optional scalar input: an empty slot is a valid
    ``None`` or the attribute fallback; a present non-constant input is not
    resolvable."""
    if len(node.inputs) > slot and node.inputs[slot]:
        arr = graph.initializers.get(node.inputs[slot])
        if arr is None:
            return False, None
        return True, float(np.asarray(arr).reshape(()))
    return True, None if fallback is None else float(fallback)


def capture_activation_params(graph: Graph, act: Node, attrs: dict) -> bool:
    """Write the activation's parameters into ``attrs``; False if a parameter
    is a runtime value that cannot be baked into generated code."""
    if act.op_type == "Clip":
        ok_lo, lo = _const_scalar(graph, act, 1, act.attr("min"))
        ok_hi, hi = _const_scalar(graph, act, 2, act.attr("max"))
        if not (ok_lo and ok_hi):
            return False
        attrs["clip_min"] = lo
        attrs["clip_max"] = hi
    elif act.op_type == "LeakyRelu":
        attrs["alpha"] = act.attr("alpha", 0.01)
    elif act.op_type == "HardSigmoid":
        attrs["alpha"] = act.attr("alpha", 0.2)
        attrs["beta"] = act.attr("beta", 0.5)
    return True


class FuseActivation(Pass):
    name = "fuse_activation"

    def run(self, graph: Graph) -> bool:
        changed = False
        prod = graph.producers()
        uses = graph.use_count()
        for act in list(graph.nodes):
            if act.op_type not in ACTIVATIONS:
                continue
            src = prod.get(act.inputs[0])
            if src is None or src.op_type not in _FUSED_NAME:
                continue
            mid = src.outputs[0]
            if uses.get(mid, 0) != 1 or mid in graph.outputs:
                continue
            attrs = dict(src.attrs)
            attrs["activation"] = act.op_type
            if not capture_activation_params(graph, act, attrs):
                continue
            fused = Node(_FUSED_NAME[src.op_type], list(src.inputs), list(act.outputs), attrs,
                         (src.name or src.op_type) + "+" + act.op_type,
                         [src.op_type, act.op_type])
            graph.nodes[graph.nodes.index(src)] = fused
            graph.remove_nodes([act])
            changed = True
        return changed
