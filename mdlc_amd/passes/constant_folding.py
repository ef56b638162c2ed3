"""Fold nodes whose inputs are all constants into new initializers.

Follows mdlc/passes/constant_folding.py:21-66: repeat until no node folds;
zero-input nodes fold only when they are ``Constant``; ``FusedElementwise`` is
never folded; a node whose constant inputs exceed ``max_numel`` elements is
left alone; a node the evaluator cannot compute is left alone.
"""

from __future__ import annotations

import numpy as np

from mdlc_amd.ir import Graph, Node
from mdlc_amd.passes.base import Pass
from mdlc_amd.passes.const_eval import evaluate

_NEVER_FOLD = {"FusedElementwise"}


class ConstantFolding(Pass):
    name = "constant_folding"

    def __init__(self, max_numel: int = 8_000_000) -> None:
        self.max_numel = max_numel

    def _foldable(self, graph: Graph, node: Node) -> bool:
        if node.op_type in _NEVER_FOLD:
            return False
        ins = node.real_inputs()
        if not ins and node.op_type != "Constant":
            return False
        if not all(graph.is_constant(e) for e in ins):
            return False
        size = sum(int(graph.initializers[e].size) for e in ins)
        return size <= self.max_numel

    def run(self, graph: Graph) -> bool:
        changed = False
        again = True
        while again:
            again = False
            for node in list(graph.nodes):
                if not self._foldable(graph, node):
                    continue
                vals = [graph.initializers[e] if e else None for e in node.inputs]
                try:
                    outs = evaluate(node, vals)
                except Exception:
                    continue
                for name, val in zip(node.outputs, outs):
                    if name:
                        graph.set_initializer(name, np.asarray(val))
                graph.remove_nodes([node])
                changed = again = True
        return changed
