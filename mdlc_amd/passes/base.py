"""Graph passes and the driver that runs them to a fixed point.

A ``Pass`` rewrites the graph in place and reports whether it changed
anything. ``PassManager`` applies its passes in sweeps until a whole sweep
changes nothing (or a sweep limit is hit), checks the graph with
``verify(graph, pass_name)`` after every change, and leaves the nodes in
topological order. The sweep-to-fixed-point contract and the default pass
order are the reference's (mdlc/passes/base.py:41-102), since they decide
which fused groups the backend receives.
"""

from __future__ import annotations

from typing import Callable, NamedTuple, Optional, Sequence

from mdlc_amd.ir import Graph


class Pass:
    """A graph rewrite. ``run`` mutates ``graph`` and returns True iff it
    changed it."""

    name: str = "pass"

    def run(self, graph: Graph) -> bool:  # pragma: no cover - interface
        raise NotImplementedError(f"{type(self).__name__}.run")


class PassRecord(NamedTuple):
    """One application of one pass."""
    name: str
    changed: bool
    nodes_before: int
    nodes_after: int


Verifier = Callable[[Graph, str], None]


class PassManager:
    def __init__(self, passes: Sequence[Pass] = (), *, max_iters: int = 8,
                 verify: Optional[Verifier] = None, verbose: bool = False,
                 history: Optional[list] = None) -> None:
        self.passes = list(passes)
        self.max_iters = max_iters
        self.verify = verify
        self.verbose = verbose
        # shared when a second manager continues the first one's record
        self.history = history if history is not None else []
        self.sweeps = 0

    def add(self, p: Pass) -> "PassManager":
        self.passes.append(p)
        return self

    def _apply(self, p: Pass, graph: Graph) -> bool:
        before = len(graph.nodes)
        changed = bool(p.run(graph))
        self.history.append(PassRecord(p.name, changed, before, len(graph.nodes)))
        if changed:
            if self.verbose:
                print(f"  [pass] {p.name}: {before} -> {len(graph.nodes)} nodes")
            if self.verify is not None:
                self.verify(graph, p.name)
        return changed

    def run(self, graph: Graph) -> Graph:
        """Sweep until a full sweep is a no-op (at most ``max_iters`` sweeps)."""
        for sweep in range(1, self.max_iters + 1):
            self.sweeps = sweep
            # every pass runs in each sweep, even after an earlier one changed
            # the graph, so a sweep is the same sequence every time
            changes = [self._apply(p, graph) for p in self.passes]
            if not any(changes):
                break
        graph.reorder_topologically()
        return graph

    def report(self) -> str:
        """Passes that changed the graph, in the order they ran."""
        rows = [f"  {r.name:24s} {r.nodes_before:3d} -> {r.nodes_after:3d}"
                for r in self.history if r.changed]
        return "\n".join(["Pass history:"] + rows)


def default_pipeline(*, verify: Optional[Verifier] = None, verbose: bool = False) -> PassManager:
    """The reference's pass order (mdlc/passes/base.py:76-102): fold
    constants, fold BatchNorm into Conv, remove dead nodes, fuse activations
    into Conv/Gemm, group the remaining pointwise chains, remove dead nodes."""
    from mdlc_amd.passes.constant_folding import ConstantFolding
    from mdlc_amd.passes.dce import DeadCodeElimination
    from mdlc_amd.passes.fuse_activation import FuseActivation
    from mdlc_amd.passes.fuse_conv_bn import FuseConvBN
    from mdlc_amd.passes.fuse_elementwise import FuseElementwise

    order = (ConstantFolding, FuseConvBN, DeadCodeElimination, FuseActivation, FuseElementwise,
             DeadCodeElimination)
    return PassManager([cls() for cls in order], verify=verify, verbose=verbose)
