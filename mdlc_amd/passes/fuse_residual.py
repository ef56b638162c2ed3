"""Fold a residual add (and the pointwise ops after it) into the conv that
feeds it, so the add runs in the conv's GEMM epilogue.

The reference stops at ``FusedElementwise`` groups (mdlc/passes/
fuse_elementwise.py); ResNet's ``Add -> Relu`` after each block and
MobileNetV2's bare residual ``Add`` stay separate memory-bound launches
there. This backend pass runs after the reference pipeline and after shape
inference. It rewrites

    y = FusedConvAct(x, w, b)            (or Conv / FusedConvBNAct)
    z = FusedElementwise[Add(y, r), act, ...](y, r)      (or a bare z = Add(y, r))

into one conv node with the same op type, ``r`` as its fourth input (the
bias slot is kept, empty when absent), output ``z``, and
``attrs["residual_subgraph"]`` / ``attrs["residual_from"]`` holding the
folded group and the name ``y`` had inside it. The group is evaluated on the
conv's output exactly as before — same float32 operations in the same
order — so every remaining tensor is bit-identical.

A member of a larger group is peeled off it the same way (the rest of the
group stays a ``FusedElementwise`` reading the conv's new output), so a
chain of residual adds folds one add per conv. The fold fires only when:
the member is an ``Add`` of ``y`` and one other tensor ``r`` of the same
shape, both from outside the group, ``r`` not depending on ``y``; the
pointwise members folded after it each read only the previous one's output,
which nothing else reads; ``y`` has no other consumer and is not a graph
output; and the conv is not depthwise (one input channel per group).
"""

from __future__ import annotations

from mdlc_amd.ir import Graph, Node
from mdlc_amd.passes.base import Pass
from mdlc_amd.passes.fuse_quant_epilogue import _descendants

CONVS = ("Conv", "FusedConvAct", "FusedConvBNAct")
POINTWISE = {"Relu", "Clip", "Sigmoid", "Tanh", "HardSwish", "HardSigmoid", "LeakyRelu"}


def _external_inputs(sub: list) -> list:
    internal = {o for n in sub for o in n.outputs if o}
    ext: list = []
    for n in sub:
        for e in n.real_inputs():
            if e not in internal and e not in ext:
                ext.append(e)
    return ext


class FuseResidualEpilogue(Pass):
    name = "fuse_residual_epilogue"

    @staticmethod
    def _depthwise(graph: Graph, conv: Node) -> bool:
        """A grouped conv with one input channel per group runs on the
        depthwise window kernel, which has no residual epilogue; other
        grouped convs run the implicit GEMM, which has."""
        if int(conv.attrs.get("group", 1)) == 1:
            return False
        w = graph.info(conv.inputs[1])
        return w is None or len(w.shape) < 2 or int(w.shape[1]) == 1

    def _peel(self, graph: Graph, grp: Node):
        """(conv, chain, y, r) for the first member of ``grp`` that is
        ``Add(y, r)`` of a foldable conv output, extended by the pointwise
        members that follow it one by one; None if there is none."""
        if grp.op_type == "Add":                     # a bare add is a one-member group
            sub, outs = [grp], list(grp.outputs)
        elif grp.op_type == "FusedElementwise":
            sub, outs = grp.attrs["subgraph"], list(grp.outputs)
        else:
            return None
        internal = {o for n in sub for o in n.outputs if o}
        prod = graph.producers()
        uses = graph.use_count()
        for i, m in enumerate(sub):
            if m.op_type != "Add" or len(m.real_inputs()) != 2 or m.inputs[0] == m.inputs[1]:
                continue
            for side in (0, 1):
                y, r = m.inputs[side], m.inputs[1 - side]
                conv = prod.get(y)
                if conv is None or conv.op_type not in CONVS or y in internal or r in internal:
                    continue
                if conv.attrs.get("residual_subgraph") or self._depthwise(graph, conv):
                    continue
                if y in graph.outputs or uses.get(y, 0) != 1:
                    continue
                if sum(y in n.inputs for n in sub) != 1:
                    continue
                yi, ri = graph.info(y), graph.info(r)
                if yi is None or ri is None or tuple(yi.shape) != tuple(ri.shape):
                    continue
                if r in _descendants(graph, y):
                    continue
                chain = [m]
                cur = m.outputs[0]
                for n in sub[i + 1:]:
                    users = [k for k in sub if cur in k.inputs]
                    if (cur in outs or users != [n] or n.op_type not in POINTWISE
                            or n.inputs[0] != cur
                            or not all(graph.is_constant(e) for e in n.inputs[1:] if e)):
                        break
                    chain.append(n)
                    cur = n.outputs[0]
                return conv, chain, y, r
        return None

    def run(self, graph: Graph) -> bool:
        changed = False
        for grp in list(graph.nodes):
            found = self._peel(graph, grp)
            if found is None:
                continue
            conv, chain, y, r = found
            z = chain[-1].outputs[0]
            ins = list(conv.inputs[:3]) + [""] * (3 - len(conv.inputs[:3])) + [r]
            attrs = dict(conv.attrs, residual_subgraph=list(chain), residual_from=y)
            fused = Node(conv.op_type, ins, [z], attrs, (conv.name or conv.op_type) + "+residual",
                         list(conv.fused_from or [conv.op_type]) + [n.op_type for n in chain])
            graph.nodes[graph.nodes.index(conv)] = fused
            rest = [] if grp.op_type == "Add" else \
                [n for n in grp.attrs["subgraph"] if all(n is not c for c in chain)]
            if rest:
                outs = [o for o in grp.outputs if o != z]
                graph.nodes[graph.nodes.index(grp)] = Node(
                    "FusedElementwise", _external_inputs(rest), outs,
                    dict(grp.attrs, subgraph=rest), grp.name, [n.op_type for n in rest])
            else:
                graph.remove_nodes([grp])
            changed = True
        if changed:
            graph.reorder_topologically()
        return changed


__all__ = ["FuseResidualEpilogue"]
