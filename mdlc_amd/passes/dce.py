"""Dead-code elimination (mdlc/passes/dce.py:9-49): keep the nodes reachable
backwards from the graph outputs, then drop unreferenced initializers and
value_info entries."""

from __future__ import annotations

from mdlc_amd.ir import Graph
from mdlc_amd.passes.base import Pass


class DeadCodeElimination(Pass):
    name = "dce"

    def run(self, graph: Graph) -> bool:
        prod = graph.producers()
        live: set = set()
        seen = set(graph.outputs)
        work = list(graph.outputs)
        while work:
            n = prod.get(work.pop())
            if n is None or id(n) in live:
                continue
            live.add(id(n))
            for e in n.real_inputs():
                if e not in seen:
                    seen.add(e)
                    work.append(e)

        n0 = len(graph.nodes)
        graph.nodes = [n for n in graph.nodes if id(n) in live]
        changed = len(graph.nodes) != n0

        referenced = set(graph.outputs) | set(graph.inputs)
        for n in graph.nodes:
            referenced.update(n.real_inputs())
            referenced.update(o for o in n.outputs if o)
        for k in [k for k in graph.initializers if k not in referenced]:
            del graph.initializers[k]
            changed = True
        for k in [k for k in graph.value_info if k not in referenced]:
            del graph.value_info[k]
        return changed
