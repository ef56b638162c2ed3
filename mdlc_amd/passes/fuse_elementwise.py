"""Group chains of pointwise ops into ``FusedElementwise`` nodes.

Legality follows mdlc/passes/fuse_elementwise.py:24-137: two pointwise nodes
join a group only across an edge that has exactly one consumer and is not a
graph output (union-find over such edges). An intermediate that something
outside the group reads becomes a group output instead of being recomputed.
A group of two or more members replaces its members at the position of its
last member; the members are kept, in graph order, in ``attrs["subgraph"]``.
"""

from __future__ import annotations

from mdlc_amd.ir import Graph, Node
from mdlc_amd.passes.base import Pass

ELEMENTWISE = {
    "Add", "Sub", "Mul", "Div",
    "Relu", "Clip", "Sigmoid", "Tanh", "HardSwish", "HardSigmoid", "LeakyRelu",
}


def _root(parent: list, i: int) -> int:
    while parent[i] != i:
        parent[i] = parent[parent[i]]
        i = parent[i]
    return i


class FuseElementwise(Pass):
    name = "fuse_elementwise"

    def run(self, graph: Graph) -> bool:
        nodes = graph.nodes
        pw = [i for i, n in enumerate(nodes) if n.op_type in ELEMENTWISE]
        if not pw:
            return False
        pos = {id(n): i for i, n in enumerate(nodes)}
        prod = graph.producers()
        uses = graph.use_count()
        cons = graph.consumers()
        exported = set(graph.outputs)

        parent = list(range(len(nodes)))
        for i in pw:
            for e in nodes[i].real_inputs():
                p = prod.get(e)
                if p is None or p.op_type not in ELEMENTWISE:
                    continue
                if uses.get(e, 0) == 1 and e not in exported:
                    ra, rb = _root(parent, pos[id(p)]), _root(parent, i)
                    if ra != rb:
                        parent[ra] = rb

        groups: dict = {}
        for i in pw:
            groups.setdefault(_root(parent, i), []).append(i)

        at: dict = {}
        gone: set = set()
        for members in groups.values():
            if len(members) < 2:
                continue
            members = sorted(members)
            inner = [nodes[i] for i in members]
            inner_ids = {id(n) for n in inner}
            made_inside = {o for n in inner for o in n.outputs if o}

            g_in: list = []
            for n in inner:
                for e in n.real_inputs():
                    if e not in made_inside and e not in g_in:
                        g_in.append(e)
            g_out: list = []
            for n in inner:
                for o in n.outputs:
                    if not o:
                        continue
                    read_outside = any(id(c) not in inner_ids for c in cons.get(o, []))
                    if o in exported or read_outside:
                        g_out.append(o)

            at[members[-1]] = Node(
                "FusedElementwise", g_in, g_out, {"subgraph": inner},
                "fused_ew_" + "_".join(str(i) for i in members),
                [n.op_type for n in inner])
            gone.update(members)

        if not at:
            return False
        graph.nodes = [at[i] if i in at else n
                       for i, n in enumerate(nodes) if i in at or i not in gone]
        return True
