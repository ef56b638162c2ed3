"""The dataflow graph container (contract of mdlc/ir/graph.py:14-190)."""

from __future__ import annotations

from collections import Counter, deque
from typing import Iterable, Iterator, Optional

import numpy as np

from mdlc_amd.ir.node import Node
from mdlc_amd.ir.tensor import DType, TensorInfo


class Graph:
    """Nodes over named edges, with constant weights held as NumPy arrays.

    ``value_info`` maps every edge name to a ``TensorInfo``; ``initializers``
    holds constant tensors. A graph input that is also an initializer is a
    constant, not a runtime feed.
    """

    def __init__(self, name: str = "graph") -> None:
        self.name = name
        self.nodes: list = []
        self.inputs: list = []
        self.outputs: list = []
        self.initializers: dict = {}
        self.value_info: dict = {}

    # -- construction -----------------------------------------------------

    def add_node(self, node: Node) -> Node:
        self.nodes.append(node)
        return node

    def set_info(self, info: TensorInfo) -> None:
        self.value_info[info.name] = info

    def info(self, name: str) -> Optional[TensorInfo]:
        return self.value_info.get(name)

    def set_initializer(self, name: str, array) -> None:
        arr = np.asarray(array)
        self.initializers[name] = arr
        try:
            dt = DType.from_numpy(arr.dtype)
        except KeyError:
            dt = DType.FLOAT32
        self.set_info(TensorInfo(name, dt, tuple(int(d) for d in arr.shape)))

    def is_constant(self, name: str) -> bool:
        return name in self.initializers

    # -- queries ------------------------------------------------------------

    @property
    def runtime_inputs(self) -> list:
        return [e for e in self.inputs if e not in self.initializers]

    def producers(self) -> dict:
        prod = {}
        for n in self.nodes:
            for o in n.outputs:
                if o:
                    prod[o] = n
        return prod

    def consumers(self) -> dict:
        cons: dict = {}
        for n in self.nodes:
            for e in n.real_inputs():
                cons.setdefault(e, []).append(n)
        return cons

    def use_count(self) -> dict:
        """Consumer slots per edge, with +1 for each graph-output mention."""
        cnt: Counter = Counter()
        for n in self.nodes:
            cnt.update(n.real_inputs())
        cnt.update(self.outputs)
        return dict(cnt)

    # -- ordering ---------------------------------------------------------

    def topo_sort(self) -> list:
        """Kahn's algorithm with a FIFO ready queue (graph.py:99-139).

        The order matters beyond validity: the memory planner walks it, so
        ties are broken exactly as the reference does — initial ready nodes
        in list order, then dependents in the order their edges were found.
        """
        avail = set(self.inputs) | set(self.initializers)
        prod = self.producers()
        index = {id(n): i for i, n in enumerate(self.nodes)}
        pending = [0] * len(self.nodes)
        waiters: list = [[] for _ in self.nodes]
        for i, n in enumerate(self.nodes):
            deps = set()
            for e in n.real_inputs():
                if e in avail:
                    continue
                p = prod.get(e)
                if p is not None:
                    deps.add(index[id(p)])
            pending[i] = len(deps)
            for d in deps:
                waiters[d].append(i)
        queue = deque(i for i in range(len(self.nodes)) if pending[i] == 0)
        out = []
        while queue:
            i = queue.popleft()
            out.append(self.nodes[i])
            for j in waiters[i]:
                pending[j] -= 1
                if pending[j] == 0:
                    queue.append(j)
        if len(out) != len(self.nodes):
            raise ValueError("graph has a cycle or dangling dependency")
        return out

    def reorder_topologically(self) -> None:
        self.nodes = self.topo_sort()

    def __iter__(self) -> Iterator[Node]:
        return iter(self.nodes)

    def __len__(self) -> int:
        return len(self.nodes)

    # -- mutation ---------------------------------------------------------

    def remove_nodes(self, gone: Iterable[Node]) -> None:
        ids = {id(n) for n in gone}
        self.nodes = [n for n in self.nodes if id(n) not in ids]

    def clone(self) -> "Graph":
        """New node objects; weight arrays are shared (treated as immutable)."""
        g = Graph(self.name)
        g.inputs = list(self.inputs)
        g.outputs = list(self.outputs)
        g.initializers = dict(self.initializers)
        g.value_info = {k: TensorInfo(v.name, v.dtype, tuple(v.shape))
                        for k, v in self.value_info.items()}
        for n in self.nodes:
            attrs = dict(n.attrs)
            if "subgraph" in attrs:
                attrs["subgraph"] = [Node(s.op_type, list(s.inputs), list(s.outputs),
                                          dict(s.attrs), s.name,
                                          None if s.fused_from is None else list(s.fused_from))
                                     for s in attrs["subgraph"]]
            g.nodes.append(Node(n.op_type, list(n.inputs), list(n.outputs), attrs, n.name,
                                None if n.fused_from is None else list(n.fused_from)))
        return g

    # -- debug ------------------------------------------------------------

    def op_histogram(self) -> dict:
        return dict(Counter(n.op_type for n in self.nodes))

    def summary(self) -> str:
        hist = ", ".join(f"{k}x{v}" for k, v in sorted(self.op_histogram().items()))
        return "\n".join([
            f"Graph {self.name!r}: {len(self.nodes)} nodes",
            f"  inputs : {', '.join(self.runtime_inputs) or '(none)'}",
            f"  outputs: {', '.join(self.outputs) or '(none)'}",
            f"  ops    : {hist}",
        ])

    def __repr__(self) -> str:
        return f"<Graph {self.name!r} nodes={len(self.nodes)}>"
