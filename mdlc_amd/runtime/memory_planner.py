"""Liveness-based buffer pooling for activations, laid out in one arena.

The assignment algorithm is the reference's (mdlc/runtime/memory_planner.py:
66-146) so buffer ids and sizes are identical: walk the topological order;
give each node's outputs a buffer before freeing its inputs; take the
smallest free buffer that fits, else grow the largest free one, else open a
new one; weights and runtime inputs are never pooled; graph outputs never
die. What this module adds for the device is placement: each buffer gets a
256-byte-aligned byte offset in a single arena, so the executor backs the
whole plan with one ``hipMalloc`` and every tensor starts on a 128-bit
(indeed 256-byte) boundary for vector loads.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from mdlc_amd.ir import Graph

ARENA_ALIGN = 256


def align_up(n: int, a: int = ARENA_ALIGN) -> int:
    return (int(n) + a - 1) // a * a


@dataclass
class Buffer:
    id: int
    size: int
    tenants: list = field(default_factory=list)


@dataclass
class MemoryPlan:
    assignment: dict
    buffers: list
    weights_bytes: int
    naive_activation_bytes: int
    planned_activation_bytes: int
    offsets: dict = field(default_factory=dict)     # buffer id -> arena byte offset
    arena_bytes: int = 0

    @property
    def reuse_ratio(self) -> float:
        if self.naive_activation_bytes == 0:
            return 1.0
        return self.planned_activation_bytes / self.naive_activation_bytes

    def offset_of(self, tensor: str) -> int:
        return self.offsets[self.assignment[tensor]]

    def report(self) -> str:
        mb = 1024 * 1024
        saved = self.naive_activation_bytes - self.planned_activation_bytes
        pct = 100.0 * saved / self.naive_activation_bytes if self.naive_activation_bytes else 0.0
        ntens = len({t for b in self.buffers for t in b.tenants})
        return "\n".join([
            "Memory plan:",
            f"  weights            : {self.weights_bytes / mb:8.3f} MB",
            f"  activations (naive): {self.naive_activation_bytes / mb:8.3f} MB  across {ntens} tensors",
            f"  activations (pool) : {self.planned_activation_bytes / mb:8.3f} MB  across {len(self.buffers)} buffers",
            f"  saved              : {saved / mb:8.3f} MB ({pct:.1f}%)",
            f"  arena (aligned)    : {self.arena_bytes / mb:8.3f} MB  align {ARENA_ALIGN} B",
        ])


def _nbytes(graph: Graph, name: str) -> int:
    info = graph.info(name)
    if info is None or not info.is_static:
        raise ValueError(f"tensor {name!r} has no static shape; run shape inference first")
    return int(info.nbytes())


def plan_memory(graph: Graph) -> MemoryPlan:
    order = graph.topo_sort()
    weights = set(graph.initializers)
    feeds = set(graph.runtime_inputs)
    outs = set(graph.outputs)

    last_use: dict = {}
    for k, n in enumerate(order):
        for e in n.real_inputs():
            last_use[e] = k
    never = len(order) + 1
    for o in outs:
        last_use[o] = never

    buffers: list = []
    free: list = []
    assignment: dict = {}
    naive = 0

    def take(name: str) -> int:
        need = _nbytes(graph, name)
        fits = [b for b in free if buffers[b].size >= need]
        if fits:
            bid = min(fits, key=lambda b: buffers[b].size)   # first smallest, in free-list order
        elif free:
            bid = max(free, key=lambda b: buffers[b].size)   # first largest; grow it
            buffers[bid].size = max(buffers[bid].size, need)
        else:
            bid = len(buffers)
            buffers.append(Buffer(bid, need))
        if bid in free:
            free.remove(bid)
        buffers[bid].tenants.append(name)
        return bid

    for k, n in enumerate(order):
        for o in n.outputs:
            if not o or o in weights or o in feeds or o in assignment:
                continue
            naive += _nbytes(graph, o)
            assignment[o] = take(o)
        for e in n.real_inputs():
            if e in weights or e in feeds or e in outs:
                continue
            if e in assignment and last_use.get(e, -1) <= k:
                bid = assignment[e]
                if bid not in free:
                    free.append(bid)

    offsets, cursor = {}, 0
    for b in buffers:
        offsets[b.id] = cursor
        cursor += align_up(b.size)
    wbytes = sum(int(a.size) * a.dtype.itemsize for a in graph.initializers.values())
    return MemoryPlan(assignment, buffers, wbytes, naive, sum(b.size for b in buffers),
                      offsets, cursor)
