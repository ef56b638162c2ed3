"""Let a global average pool write its flattened output directly.

``y = GlobalAveragePool(x)`` ([N, C, 1, 1]) followed by ``z = Flatten(y,
axis=1)`` ([N, C]) is the classifier head of both CNN families here; the
flatten is a copy launch on the device (the planner gives every tensor its
own slot, so a view cannot alias). When ``y`` feeds only the flatten and is
not a graph output, the pool produces ``z`` itself with ``attrs["flatten"]``
set: the same values in the same memory order, one launch fewer. Applies to
``GlobalAveragePool`` and ``QGlobalAveragePool`` (whose channels-last [N, C]
output is the same bytes). Runs after shape inference.
"""

from __future__ import annotations

from mdlc_amd.ir import Graph, Node
from mdlc_amd.passes.base import Pass

POOLS = ("GlobalAveragePool", "QGlobalAveragePool")


class FoldPoolFlatten(Pass):
    name = "fold_pool_flatten"

    def run(self, graph: Graph) -> bool:
        changed = False
        for pool in list(graph.nodes):
            if pool.op_type not in POOLS or pool.attrs.get("flatten"):
                continue
            y = pool.outputs[0]
            if y in graph.outputs or graph.use_count().get(y, 0) != 1:
                continue
            (fl,) = graph.consumers()[y]
            info = graph.info(y)
            if fl.op_type != "Flatten" or int(fl.attrs.get("axis", 1)) != 1 or info is None \
                    or len(info.shape) != 4 or tuple(info.shape[2:]) != (1, 1):
                continue
            fused = Node(pool.op_type, list(pool.inputs), list(fl.outputs), dict(pool.attrs, flatten=True),
                         (pool.name or pool.op_type) + "+Flatten",
                         list(pool.fused_from or [pool.op_type]) + ["Flatten"])
            graph.nodes[graph.nodes.index(pool)] = fused
            graph.remove_nodes([fl])
            changed = True
        return changed


__all__ = ["FoldPoolFlatten"]
