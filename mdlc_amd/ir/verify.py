"""Well-formedness rules for the IR, checked after every pass that changes it.

The graph is in SSA form over named values. A pass that breaks that form
(a dangling read, a value written twice, a cycle, dead work left behind)
would otherwise fail much later inside codegen or the memory planner, far
from the pass that caused it. The invariants are the ones the reference
checks (mdlc/ir/verify.py:28-83); the rule table, the acyclicity check and
the reporting (all violations at once, one line each) are this package's.

Rules, by tag:

* ``ssa``        a value is written by at most one node, and never by a node
                 when it is already a graph input or a constant;
* ``def-use``    every value a node reads, and every graph output, exists;
* ``acyclic``    no value depends on itself through node edges;
* ``dead``       every node's result is read by a node or is a graph output;
* ``const``      a constant's array has the shape recorded for it.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Iterator

from mdlc_amd.ir.graph import Graph


class GraphVerifyError(AssertionError):
    """The graph violates at least one well-formedness rule; ``violations``
    holds every one found."""

    def __init__(self, violations: list, context: str = "") -> None:
        self.violations = list(violations)
        self.context = context
        head = f"malformed graph{f' after {context}' if context else ''}"
        super().__init__(head + ": " + "; ".join(str(v) for v in self.violations))


@dataclass(frozen=True)
class Violation:
    rule: str
    message: str

    def __str__(self) -> str:
        return f"[{self.rule}] {self.message}"


def _label(node) -> str:
    return f"{node.op_type}:{node.name}" if node.name else node.op_type


def _writers(g: Graph) -> dict:
    """value -> every node that writes it, in node order."""
    out: dict = {}
    for n in g.nodes:
        for v in n.outputs:
            if v:
                out.setdefault(v, []).append(n)
    return out


def _rule_ssa(g: Graph, writers: dict) -> Iterator[Violation]:
    sources = set(g.inputs) | set(g.initializers)
    for v, ws in writers.items():
        if len(ws) > 1:
            yield Violation("ssa", f"{v!r} is written {len(ws)} times "
                                   f"(by {', '.join(_label(n) for n in ws)})")
        if v in sources:
            kind = "graph input" if v in g.inputs else "constant"
            yield Violation("ssa", f"{_label(ws[0])} overwrites {kind} {v!r}")


def _rule_def_use(g: Graph, writers: dict) -> Iterator[Violation]:
    exists = set(g.inputs) | set(g.initializers) | set(writers)
    for n in g.nodes:
        for v in n.real_inputs():
            if v not in exists:
                yield Violation("def-use", f"{_label(n)} reads {v!r}, which nothing defines")
    for v in g.outputs:
        if v not in exists:
            yield Violation("def-use", f"graph output {v!r} is never computed")


def _rule_acyclic(g: Graph, writers: dict) -> Iterator[Violation]:
    """Iterative three-colour depth-first search over node -> producer edges;
    reports one node on each cycle found."""
    WHITE, GREY, BLACK = 0, 1, 2
    colour = {id(n): WHITE for n in g.nodes}
    preds = {id(n): [w for v in n.real_inputs() for w in writers.get(v, ())] for n in g.nodes}
    for root in g.nodes:
        if colour[id(root)] != WHITE:
            continue
        stack = [(root, iter(preds[id(root)]))]
        colour[id(root)] = GREY
        while stack:
            node, it = stack[-1]
            nxt = next(it, None)
            if nxt is None:
                colour[id(node)] = BLACK
                stack.pop()
            elif colour[id(nxt)] == GREY:
                yield Violation("acyclic", f"{_label(nxt)} depends on its own output")
                colour[id(nxt)] = BLACK          # report each cycle once
            elif colour[id(nxt)] == WHITE:
                colour[id(nxt)] = GREY
                stack.append((nxt, iter(preds[id(nxt)])))


def _rule_dead(g: Graph, writers: dict) -> Iterator[Violation]:
    read = set(g.outputs)
    for n in g.nodes:
        read.update(n.real_inputs())
    for n in g.nodes:
        results = [v for v in n.outputs if v]
        if results and read.isdisjoint(results):
            yield Violation("dead", f"{_label(n)} computes {results} but nothing reads them")


def _rule_const(g: Graph, writers: dict) -> Iterator[Violation]:
    for name, arr in g.initializers.items():
        info = g.info(name)
        if info is not None and info.is_static and tuple(info.shape) != tuple(arr.shape):
            yield Violation("const", f"constant {name!r} holds shape {tuple(arr.shape)} "
                                     f"but is recorded as {tuple(info.shape)}")


RULES = (_rule_ssa, _rule_def_use, _rule_acyclic, _rule_dead, _rule_const)


def check_graph(g: Graph) -> list:
    """Every rule violation of ``g`` (empty when the graph is well formed)."""
    writers = _writers(g)
    return [v for rule in RULES for v in rule(g, writers)]


def verify_graph(g: Graph, *, context: str = "") -> None:
    """Raise ``GraphVerifyError`` listing every violation; ``context`` names
    the pass that just ran."""
    found = check_graph(g)
    if found:
        raise GraphVerifyError(found, context)
