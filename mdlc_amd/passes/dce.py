"""Dead-code elimination by reference counting.

A node is dead when no node reads any of its results and none is a graph
output. Removing a dead node releases one read of each of its operands,
which may make their producers dead in turn; a work list follows those
releases until nothing changes. On an acyclic graph this removes exactly
the nodes the graph outputs do not depend on, the same set as the
reference's backward reachability walk (mdlc/passes/dce.py:9-49). Constants
no surviving node reads, and shape records for values that no longer exist,
are dropped as well.
"""

from __future__ import annotations

from collections import Counter

from mdlc_amd.ir import Graph
from mdlc_amd.passes.base import Pass


class DeadCodeElimination(Pass):
    name = "dce"

    def run(self, graph: Graph) -> bool:
        reads: Counter = Counter(graph.outputs)      # a graph output counts as a read
        for n in graph.nodes:
            reads.update(n.real_inputs())
        writer = graph.producers()

        def is_dead(node) -> bool:
            return all(reads[v] == 0 for v in node.outputs if v)

        dead: set = set()
        work = [n for n in graph.nodes if is_dead(n)]
        while work:
            n = work.pop()
            if id(n) in dead:
                continue
            dead.add(id(n))
            for v in n.real_inputs():
                reads[v] -= 1
                w = writer.get(v)
                if reads[v] == 0 and w is not None and id(w) not in dead and is_dead(w):
                    work.append(w)

        changed = bool(dead)
        if dead:
            graph.nodes = [n for n in graph.nodes if id(n) not in dead]

        alive = set(graph.inputs) | set(graph.outputs)
        for n in graph.nodes:
            alive.update(n.real_inputs())
            alive.update(v for v in n.outputs if v)
        unused_consts = [k for k in graph.initializers if k not in alive]
        for k in unused_consts:
            graph.initializers.pop(k)
        for k in [k for k in graph.value_info if k not in alive]:
            graph.value_info.pop(k)
        return changed or bool(unused_consts)
