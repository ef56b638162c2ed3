"""The IR rules, dead-code elimination and the pass driver.

* Each malformed graph below breaks one rule, and the verifier names that
  rule; a graph with several faults reports all of them.
* Dead-code elimination keeps exactly the nodes the outputs depend on
  (checked against a brute-force dependency closure on random DAGs).
* Once the default pipeline has converged, every pass is a no-op on the
  result and the result is well formed (the fixed-point contract).
"""

from __future__ import annotations

import random

import numpy as np
import pytest

from conftest import build_graph
from mdlc_amd.ir import Graph, GraphVerifyError, Node, verify_graph
from mdlc_amd.ir.verify import check_graph
from mdlc_amd.passes import (
    ConstantFolding, DeadCodeElimination, FuseActivation, FuseConvBN, FuseElementwise, default_pipeline,
)
from mdlc_amd.passes.base import Pass, PassManager


def _graph(nodes, outputs=("y",), inputs=("x",)):
    g = Graph("case")
    g.inputs, g.outputs = list(inputs), list(outputs)
    for op, ins, outs in nodes:
        g.add_node(Node(op, list(ins), list(outs)))
    return g


def _bad_const_shape():
    g = _graph([("Add", ["x", "w"], ["y"])])
    g.set_initializer("w", np.zeros((2, 3), np.float32))
    g.value_info["w"].shape = (3, 2)
    return g


MALFORMED = {
    "read of an undefined value": (lambda: _graph([("Relu", ["ghost"], ["y"])]), "def-use"),
    "output never computed": (lambda: _graph([("Relu", ["x"], ["y"])], outputs=("y", "z")), "def-use"),
    "value written twice": (lambda: _graph([("Relu", ["x"], ["y"]), ("Neg", ["x"], ["y"])]), "ssa"),
    "input overwritten": (lambda: _graph([("Relu", ["x"], ["x"]), ("Neg", ["x"], ["y"])]), "ssa"),
    "two-node cycle": (lambda: _graph([("Add", ["x", "b"], ["a"]), ("Add", ["a", "x"], ["b"]),
                                       ("Relu", ["a"], ["y"])]), "acyclic"),
    "self loop": (lambda: _graph([("Add", ["x", "s"], ["s"]), ("Relu", ["s"], ["y"])]), "acyclic"),
    "unread result": (lambda: _graph([("Relu", ["x"], ["y"]), ("Neg", ["x"], ["unused"])]), "dead"),
    "constant of the wrong shape": (_bad_const_shape, "const"),
}


@pytest.mark.parametrize("case", sorted(MALFORMED))
def test_each_rule_is_reported(case):
    make, rule = MALFORMED[case]
    g = make()
    with pytest.raises(GraphVerifyError) as info:
        verify_graph(g, context="unit")
    assert rule in {v.rule for v in info.value.violations}, info.value
    assert "after unit" in str(info.value)


def test_every_violation_is_listed():
    g = _graph([("Relu", ["ghost"], ["y"]), ("Neg", ["x"], ["y"]), ("Exp", ["x"], ["unused"])],
               outputs=("y", "z"))
    rules = sorted(v.rule for v in check_graph(g))
    assert rules == ["dead", "def-use", "def-use", "ssa"]


def test_well_formed_graphs_pass(model_case):
    name, kw = model_case
    g, _ = build_graph(name, **kw)
    assert check_graph(g) == []


def _random_dag(rng: random.Random, n_nodes: int):
    values = ["x"]
    nodes = []
    for i in range(n_nodes):
        ins = rng.sample(values, k=min(len(values), rng.choice((1, 2))))
        out = f"v{i}"
        nodes.append(("Add" if len(ins) == 2 else "Relu", ins, [out]))
        values.append(out)
    outs = rng.sample(values[1:], k=rng.randint(1, 3))
    return nodes, outs


def _closure(nodes, outs):
    """Indices of nodes the outputs depend on (fixed-point iteration)."""
    need, keep = set(outs), set()
    grew = True
    while grew:
        grew = False
        for i, (_, ins, o) in enumerate(nodes):
            if i not in keep and o[0] in need:
                keep.add(i)
                need.update(ins)
                grew = True
    return keep


@pytest.mark.parametrize("seed", range(12))
def test_dce_keeps_exactly_the_dependencies_of_the_outputs(seed):
    rng = random.Random(seed)
    nodes, outs = _random_dag(rng, 14)
    g = _graph(nodes, outputs=outs)
    g.set_initializer("unused_w", np.ones(3, np.float32))
    changed = DeadCodeElimination().run(g)
    kept = {n.outputs[0] for n in g.nodes}
    want = {nodes[i][2][0] for i in _closure(nodes, outs)}
    assert kept == want
    assert changed and "unused_w" not in g.initializers
    assert check_graph(g) == []
    assert not DeadCodeElimination().run(g)


class _CountDown(Pass):
    """Removes one trailing identity per run until none is left."""
    name = "countdown"

    def run(self, graph):
        for n in graph.nodes:
            if n.op_type == "Identity" and n.outputs[0] != "y":
                (src,) = n.inputs
                graph.nodes.remove(n)
                for m in graph.nodes:
                    m.inputs = [src if e == n.outputs[0] else e for e in m.inputs]
                return True
        return False


def test_manager_sweeps_to_a_fixed_point_and_verifies_each_change():
    chain = [("Identity", ["x"], ["a0"])] + [("Identity", [f"a{i}"], [f"a{i + 1}"]) for i in range(4)]
    g = _graph(chain + [("Relu", ["a5"], ["y"])])
    seen = []
    pm = PassManager([_CountDown()], verify=lambda graph, name: seen.append((name, len(graph.nodes))))
    pm.run(g)
    assert [n.op_type for n in g.nodes] == ["Relu"]
    assert seen == [("countdown", k) for k in (5, 4, 3, 2, 1)]
    assert pm.sweeps == 6                           # five changing sweeps and one quiet one
    assert "countdown" in pm.report()

    g = _graph(chain + [("Relu", ["a5"], ["y"])])
    PassManager([_CountDown()], max_iters=2).run(g)
    assert len(g.nodes) == 4                       # stopped by the sweep limit


PASSES = [ConstantFolding, FuseConvBN, DeadCodeElimination, FuseActivation, FuseElementwise]


@pytest.mark.parametrize("pass_cls", PASSES, ids=lambda c: c.__name__)
def test_converged_pipeline_is_a_fixed_point_of_every_pass(pass_cls, model_case):
    name, kw = model_case
    g, _ = build_graph(name, **kw)
    g = default_pipeline(verify=lambda graph, p: verify_graph(graph, context=p)).run(g)
    before = [(n.op_type, tuple(n.inputs), tuple(n.outputs)) for n in g.nodes]
    assert not pass_cls().run(g), f"{pass_cls.__name__} changed a converged graph"
    assert [(n.op_type, tuple(n.inputs), tuple(n.outputs)) for n in g.nodes] == before
    assert check_graph(g) == []
