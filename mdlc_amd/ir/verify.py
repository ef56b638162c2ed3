"""Structural invariants of a graph, checked after every pass.

Same checks as the reference verifier (mdlc/ir/verify.py:28-83): each value
has one producer and does not shadow an input or constant, every read value is
defined, every graph output is produced, the graph is acyclic, no node is an
orphan, and initializer arrays agree with their recorded shapes.
"""

from __future__ import annotations

from mdlc_amd.ir.graph import Graph


class GraphVerifyError(AssertionError):
    """A structural invariant of the IR does not hold."""


def verify_graph(g: Graph, *, context: str = "") -> None:
    sfx = f" (after {context})" if context else ""
    known = set(g.inputs) | set(g.initializers)
    made_by: dict = {}
    for n in g.nodes:
        for o in n.outputs:
            if not o:
                continue
            if o in made_by:
                raise GraphVerifyError(
                    f"value {o!r} has two producers ({made_by[o]} and {n.op_type}){sfx}")
            if o in known:
                raise GraphVerifyError(
                    f"value {o!r} produced by {n.op_type} shadows a graph input/initializer{sfx}")
            made_by[o] = n.op_type
    known |= set(made_by)

    for n in g.nodes:
        for e in n.real_inputs():
            if e not in known:
                raise GraphVerifyError(
                    f"node {n.op_type}({n.name!r}) reads undefined value {e!r}{sfx}")

    for o in g.outputs:
        if o not in known:
            raise GraphVerifyError(f"graph output {o!r} is not produced{sfx}")

    try:
        g.topo_sort()
    except ValueError as exc:
        raise GraphVerifyError(f"{exc}{sfx}") from exc

    read = {e for n in g.nodes for e in n.real_inputs()} | set(g.outputs)
    for n in g.nodes:
        outs = [o for o in n.outputs if o]
        if outs and not any(o in read for o in outs):
            raise GraphVerifyError(
                f"orphan node {n.op_type}({n.name!r}): outputs {outs} are never consumed{sfx}")

    for name, arr in g.initializers.items():
        info = g.info(name)
        if info is not None and info.is_static and tuple(info.shape) != tuple(arr.shape):
            raise GraphVerifyError(
                f"initializer {name!r} shape {arr.shape} != recorded TensorInfo {info.shape}{sfx}")
